"""StarCoder2-8B and GPTBigCode-1B decoder harnesses that drive the quantized GEMV.

Restates the decode paths of the reference's runtime_8b.py (Starcoder2Block
:20-57, Starcoder2 :60-110) and runtime_1b.py (BigCodeBlock :17-49,
GPTBigCode :52-91), the KV-cache / graph machinery of runtime_shared.py
(CachedDecoding :345-394) and its beam sampling (_penalize/_warp/_beam_sample
:170-265). Every quantized linear is a `GGUFLinear` over SoA arrays, so each
decode step runs the HIP GEMV 4 x layers + 1 times (StarCoder2's q, k and v
are one fused linear: their SoA rows concatenated, a pure byte
concatenation; GPTBigCode's c_attn is one linear in the checkpoint already).

Two ways to run a GPU decode step (`fused` on the model):
- fused (the default): a layer's attention (rotation of q and k, the cache
  write and the attention over the cache) is one HIP kernel
  (`svq_decode_attention`), and the LayerNorms, GELU and residual adds run
  inside the GEMVs (`svq_gemv_fused`): five HIP launches per layer;
- as the reference runs it (`fused = False`): only the quantized linears are
  HIP GEMVs; LayerNorm, attention, GELU and the residual adds are the
  reference's torch ops.
Prefill and host decoding use the reference's torch ops.

Attention products are arranged so that no batched product takes a transposed
view as its right operand: decode computes K @ q^T with a contiguous q^T, and
prefill multiplies by a contiguous K^T.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from . import _native as native
from .quantization import BLOCK_BYTES, GGUFEmbedding, GGUFLinear, tied_head

# Sampling settings of the reference (runtime_shared.py:148-150).
TOP_K = 50
REPETITION_PENALTY = 3.1
LENGTH_PENALTY = -1.0


@dataclass(frozen=True)
class DecoderConfig:
    """StarCoder2-8B-style decoder shape (the reference's runtime_8b.py reads
    these from the GGUF's embedded config; rope_theta and sliding_window
    default as in runtime_8b.py:71-72)."""
    hidden: int = 4608
    heads: int = 36
    kv_heads: int = 4
    inner: int = 18432
    layers: int = 32
    vocab: int = 49152
    rope_theta: float = 1e6
    window: int = 4096
    context: int = 16000

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads


@dataclass(frozen=True)
class BigCodeConfig:
    """GPTBigCode-1B (StarVector-1B) decoder shape: multi-query attention (one
    key/value head), learned position embeddings, GELU MLP (runtime_1b.py:52-68
    reads these from the GGUF's embedded config)."""
    hidden: int = 2048
    heads: int = 16
    inner: int = 8192
    layers: int = 24
    vocab: int = 49152
    context: int = 8192

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads

    @property
    def kv_heads(self) -> int:
        return 1


def random_soa(qtype: str, n: int, k: int, generator: torch.Generator, device) -> tuple:
    """Seeded synthetic SoA arrays: uniform payload bytes (uniform codes;
    Q8_0 int8 in [-127, 127]) and fp16 scales uniform in [1e-3, 2e-2]."""
    blocks = n * k // 32
    if qtype == "Q8_0":
        q = torch.randint(-127, 128, (blocks * 32,), generator=generator, device=device,
                          dtype=torch.int8).view(torch.uint8)
    else:
        q = torch.randint(0, 256, (blocks * (BLOCK_BYTES[qtype] - 2),), generator=generator,
                          device=device, dtype=torch.uint8)
    d = torch.rand(blocks, generator=generator, device=device) * (2e-2 - 1e-3) + 1e-3
    return q, d.half().view(torch.uint8)


def random_linear(qtype, n, k, generator, device, bias=True):
    layer = GGUFLinear(k, n)
    layer.set_soa(qtype, (n, k), *random_soa(qtype, n, k, generator, device))
    if bias:
        layer.set_dense("bias", (torch.randn(n, generator=generator, device=device) * 0.02).half())
    return layer


def random_norm(width, generator, device):
    norm = nn.LayerNorm(width, eps=1e-5, device=device, dtype=torch.float16)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.05 * torch.randn(width, generator=generator, device=device))
        norm.bias.copy_(0.02 * torch.randn(width, generator=generator, device=device))
    norm.weight.requires_grad_(False)
    norm.bias.requires_grad_(False)
    return norm


def random_embedding(qtype, rows, width, generator, device):
    table = GGUFEmbedding(rows, width)
    table.set_soa(qtype, (rows, width), *random_soa(qtype, rows, width, generator, device))
    table.output_dtype = torch.float16
    return table


def rotate(x, cos, sin):
    """Rotary embedding over rotated halves (runtime_8b.py:14-17)."""
    first, second = x.chunk(2, dim=-1)
    return x * cos + torch.cat((-second, first), dim=-1) * sin


def decode_scores(keys, q, bias):
    """Decode attention probabilities of one query row per (row, key/value
    head): the reference's `baddbmm(bias, q, K^T, alpha=head_dim^-0.5)` and
    fp32 softmax (runtime_8b.py:45-48; runtime_1b.py:45-47), computed as
    K @ q^T with a contiguous q^T. keys [B, span, D], q [B, group, D];
    returns [B, group, span] in q's dtype, for a `bmm` with V."""
    hd = q.shape[-1]
    qt = q.transpose(1, 2).contiguous()
    scores = torch.bmm(keys, qt).transpose(1, 2) * hd ** -0.5 + bias
    return torch.softmax(scores, -1, dtype=torch.float32).to(q.dtype).contiguous()


class Starcoder2Block(nn.Module):
    """Grouped-query block writing its keys/values into a fixed cache
    (runtime_8b.py:20-57), with q/k/v as one fused quantized linear."""

    def __init__(self, cfg: DecoderConfig, qtype, generator, device):
        super().__init__()
        self.cfg = cfg
        hd = cfg.head_dim
        self.input_layernorm = random_norm(cfg.hidden, generator, device)
        self.qkv_proj = random_linear(qtype, cfg.hidden + 2 * cfg.kv_heads * hd, cfg.hidden,
                                      generator, device)
        self.o_proj = random_linear(qtype, cfg.hidden, cfg.hidden, generator, device)
        self.post_attention_layernorm = random_norm(cfg.hidden, generator, device)
        self.c_fc = random_linear(qtype, cfg.inner, cfg.hidden, generator, device)
        self.c_proj = random_linear(qtype, cfg.hidden, cfg.inner, generator, device)

    def forward(self, x, cos, sin, keys, values, position=None, bias=None, workspaces=None):
        """Prefill (position None) or one decode step. With `workspaces` (the
        decoding's own attention and GEMV workspaces) a GPU decode step runs
        the fused HIP layer; without, the reference's torch ops."""
        cfg = self.cfg
        hd, heads, kvh = cfg.head_dim, cfg.heads, cfg.kv_heads
        rows, length, hidden = x.shape
        if position is not None and workspaces is not None:
            # Five HIP launches per layer: the LayerNorms, GELU and residual
            # adds run inside the GEMVs; the rotation, cache write and
            # attention are one kernel (+ merge).
            x = x.reshape(rows, hidden)
            qkv = fused_linear(self.qkv_proj, x, norm=self.input_layernorm)
            out = torch.empty((rows, hidden), dtype=x.dtype, device=x.device)
            native.decode_attention(qkv, cos.view(-1), sin.view(-1), keys, values, position,
                                    None, out, heads, kvh, hd ** -0.5, workspaces["attention"],
                                    window=cfg.window)
            x = fused_linear(self.o_proj, out, residual=x)
            h = fused_linear(self.c_fc, x, norm=self.post_attention_layernorm, gelu=True)
            return fused_linear(self.c_proj, h, residual=x,
                                workspace=workspaces["gemv"]).view(rows, 1, hidden)
        qkv = self.qkv_proj(self.input_layernorm(x))
        out = self.torch_attention(qkv, cos, sin, keys, values, position, bias)
        x = x + self.o_proj(out)
        return x + self.c_proj(F.gelu(self.c_fc(self.post_attention_layernorm(x)), approximate="tanh"))

    def torch_attention(self, qkv, cos, sin, keys, values, position=None, bias=None):
        """The reference's attention ops (runtime_8b.py:38-55) in torch:
        prefill (position None) and decode on any device."""
        cfg = self.cfg
        hd, heads, kvh = cfg.head_dim, cfg.heads, cfg.kv_heads
        rows, length, _ = qkv.shape
        hidden = heads * hd
        q, k, v = qkv.split((hidden, kvh * hd, kvh * hd), -1)
        q = rotate(q.view(rows, length, heads, hd).transpose(1, 2), cos, sin)
        k = rotate(k.view(rows, length, kvh, hd).transpose(1, 2), cos, sin)
        v = v.view(rows, length, kvh, hd).transpose(1, 2)
        group = heads // kvh
        if position is None:
            keys[:, :, :length] = k
            values[:, :, :length] = v
            return causal_attention(q, k, v, group).reshape(rows, length, hidden)
        keys.index_copy_(2, position, k)
        values.index_copy_(2, position, v)
        probs = decode_scores(keys.flatten(0, 1), q.reshape(rows * kvh, group, hd), bias)
        return torch.bmm(probs, values.flatten(0, 1)).view(rows, 1, hidden)


class BigCodeBlock(nn.Module):
    """GPTBigCode multi-query block writing its keys/values into a fixed
    cache (runtime_1b.py:17-49). The cache is [rows, 1, capacity, head_dim]:
    the reference's [rows, capacity, head_dim] with its one key/value head
    kept as a dimension, the layout of the StarCoder2 cache."""

    def __init__(self, cfg: BigCodeConfig, qtype, generator, device):
        super().__init__()
        self.cfg = cfg
        hd = cfg.head_dim
        self.ln_1 = random_norm(cfg.hidden, generator, device)
        self.c_attn = random_linear(qtype, cfg.hidden + 2 * hd, cfg.hidden, generator, device)
        self.attn_proj = random_linear(qtype, cfg.hidden, cfg.hidden, generator, device)
        self.ln_2 = random_norm(cfg.hidden, generator, device)
        self.c_fc = random_linear(qtype, cfg.inner, cfg.hidden, generator, device)
        self.c_proj = random_linear(qtype, cfg.hidden, cfg.inner, generator, device)

    def forward(self, x, keys, values, position=None, bias=None, workspaces=None):
        cfg = self.cfg
        hd, heads = cfg.head_dim, cfg.heads
        rows, length, hidden = x.shape
        if position is not None and workspaces is not None:
            # Five HIP launches per layer, as the StarCoder2 block: no
            # rotation; the causal mask is the attention kernel's window,
            # wider than the span.
            x = x.reshape(rows, hidden)
            qkv = fused_linear(self.c_attn, x, norm=self.ln_1)
            out = torch.empty((rows, hidden), dtype=x.dtype, device=x.device)
            native.decode_attention(qkv, None, None, keys, values, position, None, out, heads, 1,
                                    hd ** -0.5, workspaces["attention"], window=keys.shape[2] + 1)
            x = fused_linear(self.attn_proj, out, residual=x)
            h = fused_linear(self.c_fc, x, norm=self.ln_2, gelu=True)
            return fused_linear(self.c_proj, h, residual=x,
                                workspace=workspaces["gemv"]).view(rows, 1, hidden)
        q, k, v = self.c_attn(self.ln_1(x)).split((hidden, hd, hd), -1)
        if position is None:
            keys[:, 0, :length] = k
            values[:, 0, :length] = v
            q = q.view(rows, length, heads, hd).transpose(1, 2)
            out = causal_attention(q, k[:, None], v[:, None], heads).reshape(rows, length, hidden)
        else:
            keys[:, 0].index_copy_(1, position, k)
            values[:, 0].index_copy_(1, position, v)
            # Multi-query: every head of a row attends the row's one key/value head.
            probs = decode_scores(keys[:, 0], q.view(rows, heads, hd), bias)
            out = torch.bmm(probs, values[:, 0]).view(rows, 1, hidden)
        x = x + self.attn_proj(out)
        return x + self.c_proj(F.gelu(self.c_fc(self.ln_2(x)), approximate="tanh"))


def fused_linear(linear, x, norm=None, residual=None, gelu=False, workspace=None):
    """`linear` (a GGUFLinear) on fp16 rows x [m, k] with the ops around it in
    one `svq_gemv_fused` launch: residual + gelu(linear(norm(x))), each part
    optional, rounded to fp16 after every op as the separate torch ops are.
    With a workspace and no norm, long rows split K (`svq_gemv_split`)."""
    spec = linear._specs["weight"]
    n, k = spec.shape
    if x.shape[-1] != k or x.dim() != 2:
        raise ValueError(f"expected [m, {k}] rows, got {tuple(x.shape)}")
    y = torch.empty((x.shape[0], n), dtype=torch.float16, device=x.device)
    native.gemv_fused(x.contiguous(), linear.weight, linear.weight_scales.view(torch.float16), y,
                      spec.qtype, bias=linear.unpack("bias", torch.float16, x.device),
                      ln_weight=None if norm is None else norm.weight,
                      ln_bias=None if norm is None else norm.bias,
                      ln_eps=1e-5 if norm is None else norm.eps, residual=residual,
                      activation="gelu_tanh" if gelu else None, workspace=workspace)
    return y


def causal_attention(q, k, v, group):
    """Causal GQA attention for prefill: q [B, H, T, D], k/v [B, Hkv, T, D];
    returns [B, T, H, D]. fp32 softmax; the key operand is transposed into a
    contiguous tensor before the product."""
    b, h, t, d = q.shape
    k = k.repeat_interleave(group, dim=1)
    v = v.repeat_interleave(group, dim=1).contiguous()
    kt = k.transpose(-1, -2).contiguous()
    out = torch.empty((b, h, t, d), dtype=q.dtype, device=q.device)
    mask = torch.full((t, t), float("-inf"), device=q.device).triu_(1)
    chunk = 4  # heads per product, bounds the fp32 score tensor
    for h0 in range(0, h, chunk):
        s = torch.matmul(q[:, h0:h0 + chunk].contiguous(), kt[:, h0:h0 + chunk]).float()
        p = torch.softmax(s * d ** -0.5 + mask, -1).to(q.dtype)
        out[:, h0:h0 + chunk] = torch.matmul(p, v[:, h0:h0 + chunk])
    return out.transpose(1, 2)


class _Decoder(nn.Module):
    """What the two decoders share: the host move, the decode workspaces and
    the `fused` switch of GPU decode steps."""

    # GPU decode steps run the fused HIP layer ops (True) or the reference's
    # torch ops around the HIP GEMVs (False).
    fused = True

    def _norms_and_tables(self):
        return [m for m in self.modules() if isinstance(m, (nn.LayerNorm, GGUFEmbedding))]

    def to_host(self):
        """Move to the CPU in fp32, the dtype the reference's loader uses on a
        CPU (its GGUFLinear then runs the tiled dequantize + F.linear path)."""
        self.to("cpu")
        for module in self._norms_and_tables():
            if isinstance(module, nn.LayerNorm):
                module.float()
            else:
                module.output_dtype = torch.float32
        return self

    def decode_workspaces(self, rows, capacity, device):
        """The fused decode step's workspaces, owned by one decoding: the
        attention partials for the whole cache, and the K-split partial sums
        of the longest rows (None when they run in one pass)."""
        cfg = self.cfg
        qtype = self.layers_list()[0].c_proj._specs["weight"].qtype
        attention = torch.empty(native.attention_workspace_bytes(rows, cfg.heads, cfg.kv_heads,
                                                                 capacity),
                                dtype=torch.uint8, device=device)
        need = native.gemv_workspace_bytes(rows, cfg.hidden, cfg.inner, qtype)
        gemv = torch.empty(need, dtype=torch.uint8, device=device) if need else None
        return {"attention": attention, "gemv": gemv}

    def rope_table(self, capacity, dtype, device):
        """Rotary tables of every cache slot, or None (no rotary embedding)."""
        return None


class Starcoder2Decoder(_Decoder):
    """StarCoder2-style decoder with a tied quantized embedding / head
    (runtime_8b.py:60-110), built from seeded synthetic SoA weights."""

    def __init__(self, cfg: DecoderConfig, qtype="Q4_0", head_qtype=None, seed=0, device="cuda"):
        super().__init__()
        self.cfg = cfg
        g = torch.Generator(device=device).manual_seed(seed)
        self.embed_tokens = random_embedding(head_qtype or qtype, cfg.vocab, cfg.hidden, g, device)
        self.layers = nn.ModuleList([Starcoder2Block(cfg, qtype, g, device) for _ in range(cfg.layers)])
        self.norm = random_norm(cfg.hidden, g, device)
        self.lm_head = tied_head(self.embed_tokens)
        self.context = cfg.context

    def layers_list(self):
        return list(self.layers)

    def _rope(self, positions, dtype):
        hd = self.cfg.head_dim
        inv_freq = 1.0 / (self.cfg.rope_theta ** (
            torch.arange(0, hd, 2, device=positions.device, dtype=torch.float32) / hd))
        angles = positions.float()[:, None] * inv_freq
        angles = torch.cat((angles, angles), -1)
        return angles.cos().to(dtype), angles.sin().to(dtype)

    def rope_table(self, capacity, dtype, device):
        return self._rope(torch.arange(capacity, device=device), dtype)

    def embed(self, ids):
        return self.embed_tokens(ids)

    def prefill(self, embeddings, rows, capacity):
        """Encode the prompt once (batch 1); its cache serves all `rows`."""
        cfg = self.cfg
        length = embeddings.shape[1]
        shape = (cfg.layers, rows, cfg.kv_heads, capacity, cfg.head_dim)
        # Keys and values in one allocation, so a beam reorder is one launch.
        kv = torch.zeros((2,) + shape, device=embeddings.device, dtype=embeddings.dtype)
        keys, values = kv[0], kv[1]
        cos, sin = self._rope(torch.arange(length, device=embeddings.device), embeddings.dtype)
        x = embeddings
        for layer, lk, lv in zip(self.layers, keys, values):
            x = layer(x, cos, sin, lk, lv)
        logits = self.lm_head(self.norm(x[:, -1]))
        return CachedDecoding(self, keys, values, length, kv), logits.expand(rows, -1)

    def decode(self, tokens, position, keys, values, span, rope=None, workspaces=None):
        """One token per row at `position`, attending the first `span` slots.
        `rope`: (cos, sin) tables over all cache slots (`_rope` of every
        position, computed once), or None to compute this position's.
        `workspaces`: the fused HIP step's (GPU), or None for the reference's
        torch ops."""
        fused = workspaces is not None and keys.is_cuda
        bias = None  # the fused attention kernel masks from the position and the window
        if not fused:
            slots = torch.arange(span, device=keys.device)
            hidden_slots = (slots > position) | (slots <= position - self.cfg.window)
            bias = torch.zeros(span, device=keys.device, dtype=keys.dtype).masked_fill_(
                hidden_slots, float("-inf"))
        if rope is None:
            cos, sin = self._rope(position, keys.dtype)
        else:  # the same elementwise values, gathered
            cos, sin = rope[0].index_select(0, position), rope[1].index_select(0, position)
        x = self.embed_tokens(tokens)[:, None]
        ws = workspaces if fused else None
        for layer, lk, lv in zip(self.layers, keys, values):
            x = layer(x, cos, sin, lk[:, :, :span], lv[:, :, :span], position, bias, ws)
        if fused:
            return fused_linear(self.lm_head, x[:, 0], norm=self.norm)
        return self.lm_head(self.norm(x[:, 0]))


class GPTBigCodeDecoder(_Decoder):
    """GPTBigCode (StarVector-1B) decoder with a tied quantized token
    embedding / head and learned position embeddings (runtime_1b.py:52-91),
    built from seeded synthetic SoA weights. `embed_qtype` is the token and
    position tables' type (the reference's converter keeps them Q8_0 in
    Q4_0 / Q5_0 files, tools/starvector_safetensors_to_gguf.py:156-159)."""

    def __init__(self, cfg: BigCodeConfig, qtype="Q4_0", embed_qtype=None, seed=0,
                 device="cuda"):
        super().__init__()
        self.cfg = cfg
        g = torch.Generator(device=device).manual_seed(seed)
        eq = embed_qtype or qtype
        self.wte = random_embedding(eq, cfg.vocab, cfg.hidden, g, device)
        self.wpe = random_embedding(eq, cfg.context, cfg.hidden, g, device)
        self.h = nn.ModuleList([BigCodeBlock(cfg, qtype, g, device) for _ in range(cfg.layers)])
        self.ln_f = random_norm(cfg.hidden, g, device)
        self.lm_head = tied_head(self.wte)
        self.context = cfg.context

    def layers_list(self):
        return list(self.h)

    def embed(self, ids):
        return self.wte(ids)

    def prefill(self, embeddings, rows, capacity):
        """Encode the prompt once (batch 1); its cache serves all `rows`."""
        cfg = self.cfg
        length = embeddings.shape[1]
        shape = (cfg.layers, rows, 1, capacity, cfg.head_dim)
        kv = torch.zeros((2,) + shape, device=embeddings.device, dtype=embeddings.dtype)
        keys, values = kv[0], kv[1]
        x = embeddings + self.wpe(torch.arange(length, device=embeddings.device))
        for block, lk, lv in zip(self.h, keys, values):
            x = block(x, lk, lv)
        logits = self.lm_head(self.ln_f(x[:, -1]))
        return CachedDecoding(self, keys, values, length, kv), logits.expand(rows, -1)

    def decode(self, tokens, position, keys, values, span, rope=None, workspaces=None):
        """One token per row at `position`, attending the first `span` slots
        (runtime_1b.py:84-91); `workspaces` as Starcoder2Decoder.decode."""
        fused = workspaces is not None and keys.is_cuda
        bias = None
        if not fused:
            slots = torch.arange(span, device=keys.device)
            bias = torch.zeros(span, device=keys.device, dtype=keys.dtype).masked_fill_(
                slots > position, float("-inf"))
        x = (self.wte(tokens) + self.wpe(position))[:, None]
        ws = workspaces if fused else None
        for block, lk, lv in zip(self.h, keys, values):
            x = block(x, lk[:, :, :span], lv[:, :, :span], position, bias, ws)
        if fused:
            return fused_linear(self.lm_head, x[:, 0], norm=self.ln_f)
        return self.lm_head(self.ln_f(x[:, 0]))


class CachedDecoding:
    """KV cache and graph-captured decode steps of one generation call
    (runtime_shared.py:345-394): one HIP graph per power-of-two span of at
    least 512 slots, captured after an eager warm-up on a side stream. The
    decoding owns the workspaces its fused steps use, so graphs captured with
    them stay valid for its whole life."""

    def __init__(self, model, keys, values, length, kv=None):
        """`kv`: the [2, ...] tensor whose halves are `keys` and `values`, if
        they share one allocation."""
        self.model, self.keys, self.values, self.length = model, keys, values, length
        self.kv = kv
        self.tokens = torch.zeros(keys.shape[1], dtype=torch.long, device=keys.device)
        self.position = torch.full((1,), length, dtype=torch.long, device=keys.device)
        self.graphs = {}
        capacity = keys.shape[3]
        # Tables of every cache slot, once (a decode step gathers its row).
        self.rope = model.rope_table(capacity, keys.dtype, keys.device)
        self.workspaces = None
        if keys.is_cuda and model.fused:
            # Allocated here, outside any capture, for the largest span.
            self.workspaces = model.decode_workspaces(keys.shape[1], capacity, keys.device)

    def span(self):
        return min(self.keys.shape[-2], max(512, 1 << self.length.bit_length()))

    def _decode(self, span):
        return self.model.decode(self.tokens, self.position, self.keys, self.values, span,
                                 self.rope, self.workspaces)

    def step(self, tokens):
        """One decode step for `tokens` [rows] (None: already in self.tokens)."""
        span = self.span()
        if tokens is not None:
            self.tokens.copy_(tokens)
        if self.keys.device.type != "cuda":
            logits = self._decode(span)
        else:
            if span not in self.graphs:
                stream = torch.cuda.Stream()
                stream.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(stream):
                    self._decode(span)  # warm-up; rewrites only this step's cache slot
                torch.cuda.current_stream().wait_stream(stream)
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, capture_error_mode="thread_local"):
                    output = self._decode(span)
                self.graphs[span] = graph, output
            graph, logits = self.graphs[span]
            graph.replay()
        self.position += 1
        self.length += 1
        return logits

    def reorder(self, parents):
        """Give every row the cache of its parent beam (runtime_shared.py:388-394).
        A row whose parent is not itself being overwritten is copied slice to
        slice (one read and one write of its cache); rows that exchange caches
        gather their sources first, as indexing with the parent list does."""
        moves = [(row, parent) for row, parent in enumerate(parents) if parent != row]
        if not moves:
            return
        n = self.length
        targets = {row for row, _ in moves}
        if any(parent in targets for _, parent in moves):
            rows = [row for row, _ in moves]
            sources = [parent for _, parent in moves]
            for cache in (self.keys, self.values):
                cache[:, rows, :, :n] = cache[:, sources, :, :n]
            return
        for row, parent in moves:
            for cache in (self.keys, self.values):
                cache[:, row, :, :n].copy_(cache[:, parent, :, :n])

    def reorder_rows(self, parents):
        """`reorder` with the parents as a device int64 tensor [rows]: on the
        GPU one kernel (svq_cache_reorder; one per cache if keys and values
        are separate allocations) moves the rows whose parent differs, with no
        host round trip; on the host it reads the parents and calls
        `reorder`."""
        if self.keys.is_cuda:
            caches = (self.keys, self.values) if self.kv is None else \
                (self.kv.view(-1, *self.kv.shape[2:]),)  # both, as 2 x layers planes
            for cache in caches:
                native.cache_reorder(cache, parents, self.length)
        else:
            self.reorder(parents.tolist())


def penalize(scores, seen):
    """Repetition penalty over generated tokens (runtime_shared.py:170-173)."""
    penalized = torch.where(scores < 0, scores * REPETITION_PENALTY, scores / REPETITION_PENALTY)
    return torch.where(seen, penalized, scores)


def warp(scores, temperature, top_p, keep):
    """Temperature, top-k and top-p warpers, in that order (runtime_shared.py:176-187)."""
    if temperature != 1.0:
        scores = scores / temperature
    threshold = torch.topk(scores, max(TOP_K, keep))[0][..., -1:]
    scores = scores.masked_fill(scores < threshold, float("-inf"))
    if top_p < 1.0:
        ordered, order = torch.sort(scores, descending=False)
        remove = ordered.softmax(-1).cumsum(-1) <= 1 - top_p
        remove[..., -keep:] = False
        scores = scores.masked_fill(remove.scatter(-1, order, remove), float("-inf"))
    return scores


def possible_draws(probs):
    """Number of probabilities > 0 as a 0-d int64 tensor, or -1 when any is
    NaN. The reference draws min(2 * beams, count_nonzero(probs)) samples
    (runtime_shared.py:232); its torch.multinomial rejects NaN input, so a NaN
    must reach multinomial rather than count as a possible draw."""
    count = (probs > 0).sum()
    return torch.where(torch.isnan(probs).any(), torch.full_like(count, -1), count)


def stable_descending(values):
    """(sorted values, order) of a 1-D tensor, descending and stable --
    `sorted(range(n), key=values.__getitem__, reverse=True)` in the
    reference's survivor selection."""
    return torch.sort(values, descending=True, stable=True)


def multinomial_draws(probs, n, noise=None):
    """`torch.multinomial(probs, n)` without replacement as PyTorch computes
    it -- the exponential race: the n largest of probs / q with q ~ Exp(1)
    drawn from the default generator (argmax for n = 1) -- so the draws are
    the same, without its input checks (the max, min and sum of probs, read
    back to the host twice). `probs` here is a softmax output, finite and
    non-negative by construction; n < 1 goes to torch.multinomial, which
    rejects it as the reference's call would. `noise`: the Exp(1) draws, if
    the caller has made them already (`torch.empty_like(probs).exponential_()`)."""
    if n < 1:
        return torch.multinomial(probs, n)
    q = torch.empty_like(probs).exponential_() if noise is None else noise
    q = probs / q
    if n == 1:
        return torch.argmax(q, -1, keepdim=True)
    return torch.topk(q, n).indices


# Candidates kept per row by `warp_candidates`: the top-k plus room for values
# tied with the k-th largest.
TIE_ROOM = 14


def warp_candidates(scores, temperature, top_p, keep, with_index=False):
    """`warp` computed on each row's top-k candidates instead of the whole
    vocabulary: the same temperature, top-k threshold and top-p removal
    (runtime_shared.py:176-187), where the reference's full-vocabulary sort,
    softmax and cumulative sum become ones over about 64 values per row.
    Every entry below the k-th largest value is -inf in both, and softmax and
    cumulative sum over the ascending order only add exact zeros for them, so
    the results match except (a) where a cumulative probability lies within
    float rounding of 1 - top_p (the two sums add in different orders) and
    (b) in the order of equal candidates.

    Returns (warped scores, overflow): overflow is a 0-d bool tensor that is
    True when a row may hold more values tied with the k-th largest than the
    candidate set has room for; the caller then uses `warp`. With
    `with_index`, also the candidates' indices [rows, candidates]: every
    entry outside them is -inf."""
    k = max(TOP_K, keep)
    vocab = scores.shape[-1]
    if k > vocab:  # the reference's top-k rejects it: same error
        out = warp(scores, temperature, top_p, keep), torch.zeros((), dtype=torch.bool)
        return out + (None,) if with_index else out
    if temperature != 1.0:
        scores = scores / temperature
    kc = min(k + TIE_ROOM, vocab)
    values, index = torch.topk(scores, kc)  # descending
    threshold = values[..., k - 1:k]
    values = values.masked_fill(values < threshold, float("-inf"))
    if kc < vocab:
        overflow = (values[..., -1] == threshold[..., 0]).any()
    else:
        overflow = torch.zeros((), dtype=torch.bool, device=scores.device)
    if top_p < 1.0:
        ascending = values.flip(-1)
        remove = ascending.softmax(-1).cumsum(-1) <= 1 - top_p
        remove[..., -keep:] = False
        values = values.masked_fill(remove.flip(-1), float("-inf"))
    out = torch.full_like(scores, float("-inf")).scatter_(-1, index, values)
    return (out, overflow, index) if with_index else (out, overflow)


def beam_steps(decoder, embeddings, steps, beams=2, temperature=1.5, top_p=0.9, capacity=None,
               on_prefill=None, on_step=None):
    """Beam sampling (runtime_shared.py:214-265) for a fixed number of decode
    steps: every step samples 2 * beams continuations from all beams, keeps
    the best `beams`, reorders the cache and decodes. The warpers run on each
    row's top-k candidates (`warp_candidates`), or on the whole vocabulary
    (`warp`) when ties at the top-k threshold overflow the candidate set.
    End-of-sequence tokens do not stop it, so every call performs exactly
    `steps` decode steps. `on_prefill()` runs after the prefill and
    `on_step(i)` after decode step i.

    The selection of the surviving beams stays on the device: parents,
    tokens and running scores are device tensors that feed the cache
    reorder, the seen-token mask and the next step directly, so a step reads
    back only the number of possible samples (`count_nonzero`, which the
    reference also reads before sampling). On the GPU two kernels
    (`svq_beam_candidates`) form each row's candidates, scores and joint
    probabilities from the logits -- their sums add in another order than
    torch's reductions, so scores agree with the torch formulation to
    rounding -- and one (`svq_beam_select`) makes the draws, the stable
    descending survivor order, the parents and tokens and the next seen rows;
    the multinomial sampling's Exp(1) draws come from the default generator
    before the host read (nothing else draws in between, so the stream of
    draws is the same).
    The token sequences are rebuilt from the per-step parents and tokens at
    the end. Returns (best token sequence, per-step running scores)."""
    keep = 2 * beams
    capacity = capacity or embeddings.shape[1] + steps + 1
    decoding, logits = decoder.prefill(embeddings, beams, capacity)
    if on_prefill is not None:
        on_prefill()
    device, vocab = logits.device, logits.shape[-1]
    on_gpu = device.type == "cuda"
    running_t = torch.tensor([0.0] + [-1e9] * (beams - 1), device=device)
    # Two seen buffers (the next step's rows are gathered from the current
    # ones), rows padded to 16 bytes for the selection kernel's copies.
    pitch = (vocab + 15) // 16 * 16
    seen_rows = [torch.zeros((beams, pitch), dtype=torch.bool, device=device) for _ in range(2)]
    beam_index = torch.arange(beams, device=device)
    history = torch.empty((steps, 2, beams), dtype=torch.long, device=device)
    # On the GPU the candidates come from one kernel pair (svq_beam_candidates)
    # when the top-k candidate set fits it.
    k = max(TOP_K, 2)
    kc = min(k + TIE_ROOM, vocab)
    device_sampling = on_gpu and k <= kc <= 64 and vocab <= 65536 and beams <= 8 and \
        logits.dtype == torch.float16
    if device_sampling:
        cand = torch.empty((beams, kc), dtype=torch.long, device=device)
        cand_scores = torch.empty((beams, kc), device=device)
        cand_probs = torch.empty(beams * kc, device=device)
        status = torch.empty(2 + beams, dtype=torch.long, device=device)
        cand_ws = native.beam_candidates_workspace(beams, vocab, kc, device)
    for step in range(steps):
        seen_now, seen_next = seen_rows[step % 2], seen_rows[1 - step % 2]
        if device_sampling:
            native.beam_candidates(logits.contiguous(), seen_now, running_t, k, kc, 2,
                                   REPETITION_PENALTY, temperature, top_p, cand, cand_scores,
                                   cand_probs, status, cand_ws)
            noise = torch.empty((1, beams * vocab), device=device).exponential_()
            possible, overflow = status[:2].tolist()  # possible -1: a NaN probability
        else:
            penalized = penalize(torch.log_softmax(logits.float(), -1), seen_now[:, :vocab])
            log_probs, overflow, candidates = warp_candidates(penalized, temperature, top_p, 2,
                                                              with_index=True)
            scores = (log_probs + running_t[:, None]).view(1, -1)
            probs = scores.softmax(-1)
            noise = torch.empty_like(probs).exponential_()
            # One host read for the sample count and the tie check. Only the
            # candidates can have a non-zero probability: count those.
            possible = possible_draws(probs.view(beams, vocab).gather(1, candidates))
            possible, overflow = torch.stack((possible, overflow.long())).tolist()
        if overflow:
            penalized = penalize(torch.log_softmax(logits.float(), -1), seen_now[:, :vocab])
            log_probs = warp(penalized, temperature, top_p, 2)
            scores = (log_probs + running_t[:, None]).view(1, -1)
            probs = scores.softmax(-1)
            possible = int(possible_draws(probs))
        draws = min(keep, possible)
        if draws < 1:
            # No possible continuation, or a NaN probability: torch.multinomial
            # raises its own error, as in the reference (which draws
            # min(keep, count_nonzero) samples from the same probabilities).
            torch.multinomial(cand_probs.view(1, -1) if device_sampling and not overflow else probs,
                              max(draws, 1) if possible < 0 else draws)
            raise RuntimeError("beam sampling: no possible continuation")
        parents, tokens = history[step, 0], history[step, 1]
        if on_gpu and not overflow and draws >= 1:
            if device_sampling:
                native.beam_select(cand_probs, noise, cand_scores, cand, draws, seen_now,
                                   seen_next, running_t, parents, tokens, decoding.tokens)
            else:
                native.beam_select(probs, noise, scores, candidates, draws, seen_now, seen_next,
                                   running_t, parents, tokens, decoding.tokens)
            next_tokens = None  # already in the step's input
        else:
            picks = multinomial_draws(probs, draws, noise)[0]
            picked = scores[0].gather(0, picks)
            # sorted(range(n), key=picked, reverse=True)[:beams]: descending, stable.
            ordered, order = stable_descending(picked)
            kept = min(beams, picks.numel())
            chosen = picks[order[:kept]]
            survivors = ordered[:kept]
            if kept < beams:  # the reference repeats its best pick and scores the rest -1e9
                chosen = torch.cat((chosen, chosen[:1].expand(beams - kept)))
                survivors = torch.cat((survivors, torch.full((beams - kept,), -1e9, device=device)))
            running_t.copy_(survivors)
            parents.copy_(chosen // vocab)
            tokens.copy_(chosen % vocab)
            seen_next.copy_(seen_now[parents])
            seen_next[beam_index, tokens] = True
            next_tokens = tokens
        decoding.reorder_rows(parents)
        logits = decoding.step(next_tokens)
        if on_step is not None:
            on_step(step + 1)
    # The token sequences: follow each final beam back through its parents.
    if not steps:
        return [], running_t.tolist()
    parents_all = history[:, 0].tolist()
    tokens_all = history[:, 1].tolist()
    beam, best = 0, []
    for step in range(steps - 1, -1, -1):
        best.append(tokens_all[step][beam])
        beam = parents_all[step][beam]
    return best[::-1], running_t.tolist()


def beam_steps_reference(decoder, embeddings, steps, beams=2, temperature=1.5, top_p=0.9,
                         capacity=None, on_prefill=None, on_step=None):
    """The reference's beam sampling loop (runtime_shared.py:214-265) for a
    fixed number of decode steps, as it runs it: the whole-vocabulary warpers
    (`warp`), `torch.multinomial` over min(2 * beams, count_nonzero) samples,
    the survivors chosen with Python's `sorted` on the host, a host list of
    parents for the cache reorder, then the next step. No end-of-sequence
    token stops it (there is no tokenizer), so the finished-beam bookkeeping
    never runs. Returns (best token sequence, running scores)."""
    keep = 2 * beams
    capacity = capacity or embeddings.shape[1] + steps + 1
    decoding, logits = decoder.prefill(embeddings, beams, capacity)
    if on_prefill is not None:
        on_prefill()
    device, vocab = logits.device, logits.shape[-1]
    running = [[] for _ in range(beams)]
    running_scores = [0.0] + [-1e9] * (beams - 1)
    seen = torch.zeros((beams, vocab), dtype=torch.bool, device=device)
    rows = torch.arange(beams, device=device)
    for step in range(steps):
        log_probs = warp(penalize(torch.log_softmax(logits.float(), -1), seen), temperature,
                         top_p, 2)
        scores = (log_probs + torch.tensor(running_scores, device=device)[:, None]).view(1, -1)
        probs = scores.softmax(-1)
        picks = torch.multinomial(probs, min(keep, int(torch.count_nonzero(probs))))
        picked = scores.gather(1, picks)[0].tolist()
        parents, tokens = zip(*(divmod(pick, vocab) for pick in picks[0].tolist()))
        order = sorted(range(len(picked)), key=picked.__getitem__, reverse=True)[:beams]
        running_scores = [picked[j] for j in order] + [-1e9] * (beams - len(order))
        order += [order[0]] * (beams - len(order))
        running = [running[parents[j]] + [tokens[j]] for j in order]
        selected = torch.tensor([parents[j] for j in order], device=device)
        next_tokens = torch.tensor([tokens[j] for j in order], device=device)
        seen = seen[selected]
        seen[rows, next_tokens] = True
        decoding.reorder([parents[j] for j in order])
        logits = decoding.step(next_tokens)
        if on_step is not None:
            on_step(step + 1)
    return running[0], running_scores
