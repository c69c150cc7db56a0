// Survivor selection of one beam-sampling step, once the number of draws is
// known (runtime_shared.py:233-262 with the loop's fixed step count):
// 1. the draws: `torch.multinomial(probs, draws)` without replacement, which
//    PyTorch computes as the exponential race -- the `draws` largest of
//    probs / noise, noise ~ Exp(1), in descending order (argmax for one
//    draw). Only the candidate tokens of each beam can have a non-zero
//    probability, so the race runs over them: `noise` is the caller's
//    Exp(1) tensor over the whole [beams * vocab], as multinomial draws it;
// 2. `sorted(range(draws), key=picked, reverse=True)[:beams]` over the drawn
//    scores (descending, stable), padded with the first survivor and
//    running score -1e9 when fewer than `beams` were drawn;
// 3. parent beam and token of each survivor (divmod by vocab);
// 4. the seen-token rows: seen_out[b] = seen_in[parent[b]] with token[b] set
//    (`seen = seen[selected]; seen[arange(beams), next_tokens] = True`).
// Every step is exact (one fp32 division per candidate, comparisons and
// copies). Every workgroup repeats the selection (at most 1024 candidates)
// and copies its share of the seen rows; workgroup 0 writes the survivors.
#include "svq_device.h"
#include "svq_launch.h"

namespace svq {

namespace {

constexpr int kThreads = 256;
constexpr int kPerLane = kBeamMaxCandidates / 64;  // candidates per lane of wave 0
constexpr int kSeenPieces = 4;                     // 16-byte seen pieces per thread
constexpr int kMaxDraws = 2 * kBeamMaxRows;

// (q, flat index) order of the race: larger q first, then the smaller index
// (argmax's first maximum).
__device__ __forceinline__ bool ahead(float q1, int64_t f1, float q2, int64_t f2) {
  return q1 > q2 || (q1 == q2 && f1 < f2);
}

__global__ __launch_bounds__(kThreads) void beam_select_kernel(BeamSelectArgs a) {
  __shared__ float qv[kBeamMaxCandidates];
  __shared__ int64_t fl[kBeamMaxCandidates];
  __shared__ int64_t chosen[kBeamMaxRows];
  const int tid = threadIdx.x;
  const int total = a.beams * a.ncand;
  for (int e = tid; e < total; e += kThreads) {
    const int b = e / a.ncand;
    // A token id outside [0, vocab) is clamped (kept in bounds, not checked).
    const int64_t t = a.candidates[e];
    const int64_t f = (int64_t)b * a.vocab + (t < 0 ? 0 : t >= a.vocab ? a.vocab - 1 : t);
    fl[e] = f;
    // A NaN race value (NaN probability, or 0 / 0) ranks last, as -inf: every
    // round then has a winner among the `draws` <= beams * ncand entries.
    const float qe = a.probs[a.compact ? e : f] / a.noise[f];
    qv[e] = qe == qe ? qe : -INFINITY;
  }
  __syncthreads();

  // Wave 0: `draws` rounds of the race's maximum over the entries not yet
  // drawn; lane l owns entries l, l + 64, ... (held in registers).
  __shared__ int64_t dpick[kMaxDraws];
  __shared__ int dslot[kMaxDraws];
  __shared__ float dscore[kMaxDraws];
  if (tid < 64) {
    const int lane = tid;
    float q[kPerLane];
    int64_t f[kPerLane];
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) {
      const int e = lane + 64 * i;
      q[i] = e < total ? qv[e] : -INFINITY;
      f[i] = e < total ? fl[e] : INT64_MAX;
    }
    uint32_t taken = 0;
    for (int d = 0; d < a.draws; ++d) {
      float bq = -INFINITY;
      int64_t bf = INT64_MAX;
      int be = -1;
#pragma unroll
      for (int i = 0; i < kPerLane; ++i)
        if (!(taken >> i & 1u) && ahead(q[i], f[i], bq, bf)) {
          bq = q[i];
          bf = f[i];
          be = lane + 64 * i;
        }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        const float oq = __shfl_xor(bq, off, 64);
        const int64_t of = __shfl_xor(bf, off, 64);
        const int oe = __shfl_xor(be, off, 64);
        if (ahead(oq, of, bq, bf)) {
          bq = oq;
          bf = of;
          be = oe;
        }
      }
      if (be < 0) {  // unreachable with NaN ranked as -inf; keeps indexes in range
        bf = fl[0];
        be = 0;
      }
      // Every lane holds the winner; its owner marks it drawn.
#pragma unroll
      for (int i = 0; i < kPerLane; ++i) taken |= (uint32_t)(f[i] == bf) << i;
      if (lane == 0) {
        dpick[d] = bf;
        dslot[d] = be;
      }
    }
  }
  __syncthreads();
  // The drawn entry's score: by flat index, or by its candidate slot.
  if (tid < a.draws) dscore[tid] = a.scores[a.compact ? dslot[tid] : dpick[tid]];
  __syncthreads();
  // Stable descending order of the drawn scores: draw i goes to its rank.
  if (tid < a.draws) {
    const float mine = dscore[tid];
    int rank = 0;
    for (int j = 0; j < a.draws; ++j) rank += dscore[j] > mine || (dscore[j] == mine && j < tid);
    if (rank < a.beams) {
      chosen[rank] = dpick[tid];
      if (blockIdx.x == 0) a.running[rank] = mine;
    }
  }
  __syncthreads();
  const int kept = min(a.beams, a.draws);
  if (tid >= kept && tid < a.beams) {
    chosen[tid] = chosen[0];
    if (blockIdx.x == 0) a.running[tid] = -1e9f;
  }
  __syncthreads();
  if (blockIdx.x == 0 && tid < a.beams) {
    const int64_t parent = chosen[tid] / a.vocab, token = chosen[tid] - parent * a.vocab;
    a.parents[tid] = parent;
    a.tokens[tid] = token;
    if (a.tokens_copy) a.tokens_copy[tid] = token;
  }

  // Seen rows: 16-byte pieces, kSeenPieces per thread, kThreads apart.
  const int64_t row_pieces = a.seen_pitch / 16;
  const int64_t base = (int64_t)blockIdx.x * kThreads * kSeenPieces + tid;
  u32x4 v[kSeenPieces];
#pragma unroll
  for (int i = 0; i < kSeenPieces; ++i) {
    const int64_t c = base + (int64_t)i * kThreads;
    if (c < a.beams * row_pieces) {
      const int b = (int)(c / row_pieces);
      const int64_t off = c - b * row_pieces;
      const int64_t parent = chosen[b] / a.vocab;
      v[i] = *reinterpret_cast<const u32x4*>(a.seen_in + parent * a.seen_pitch + off * 16);
    }
  }
#pragma unroll
  for (int i = 0; i < kSeenPieces; ++i) {
    const int64_t c = base + (int64_t)i * kThreads;
    if (c < a.beams * row_pieces) {
      const int b = (int)(c / row_pieces);
      const int64_t off = c - b * row_pieces;
      const int64_t parent = chosen[b] / a.vocab;
      const int64_t at = chosen[b] - parent * a.vocab - off * 16;  // token byte in this piece
      if (at >= 0 && at < 16) {
        uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
        w[at / 4] |= 1u << (8 * (at % 4));
        v[i].x = w[0]; v[i].y = w[1]; v[i].z = w[2]; v[i].w = w[3];
      }
      *reinterpret_cast<u32x4*>(a.seen_out + b * a.seen_pitch + off * 16) = v[i];
    }
  }
}

// ---------------------------------------------------------------------------
// Candidates of a beam-sampling step (runtime_shared.py:228-231: log-softmax,
// repetition penalty, temperature, top-k and top-p warpers, running scores
// and the joint softmax over all beams), computed on each row's kc largest
// warped log-probabilities instead of the whole vocabulary:
//   lp = log_softmax(x) = (x - max) - log(sum exp(x - max))  (expf / logf);
//   w = penalty: seen ? (lp < 0 ? lp * p : lp / p) : lp;  v = w / t
//   (temperature t; no division at t = 1).
// w is increasing in x among the unseen tokens and among the seen ones, so
// the kc largest w lie among the kc largest x of each class, and v is
// monotone in w (ties that the division creates at the kc-th value only
// matter where that value is also the k-th, which is reported as overflow).
// 1. Slice kernel (16 slices of 4096 tokens per row at most, 256 threads):
//    the slice's max and sum of exp(x - max), and its kc largest x among
//    unseen and among seen tokens (radix select on order-preserving keys;
//    ties at the cut keep the first in thread order).
// 2. Merge kernel (one workgroup per row): the row's max and log-sum from
//    the slices' (rescaled in slice order), w and v of every kept entry, the
//    kc largest w, sorted on v descending (token ascending); top-k: values
//    below the k-th become -inf; top-p over the kc values: softmax, sums
//    from the smallest up, removal where the sum <= 1 - top_p except the
//    `keep` largest; candidate score = v + running[row].
// 3. Joint kernel (one workgroup): softmax over all candidates of all rows,
//    the number of non-zero probabilities and the overflow flag.
// The sums add in another order than torch's reductions (the results agree
// to rounding); comparisons, the penalty, the temperature and the score
// additions are the same fp32 operations.
constexpr int kSliceThreads = 256;
constexpr int kSliceJ = 16;                          // tokens per thread
constexpr int kSliceLen = kSliceThreads * kSliceJ;   // 4096
constexpr int kMaxSlices = kCandMaxVocab / kSliceLen;  // 16
constexpr int kCandThreads = 1024;
constexpr int kMergeJ = 2 * kMaxSlices * kCandMax / kCandThreads;  // entries per thread: 2

__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t b = __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Block-wide max / sum over T threads, the same order every call.
template <int T>
__device__ __forceinline__ float block_reduce(float v, bool is_max, float* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float o = __shfl_xor(v, off, 64);
    v = is_max ? fmaxf(v, o) : v + o;
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();  // `red` free for reuse
  if (lane == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < T / 64; ++i) r = is_max ? fmaxf(r, red[i]) : r + red[i];
  return r;
}

// Exclusive prefix sum over the threads of a T-thread workgroup (thread
// order), and the total.
template <int T>
__device__ __forceinline__ uint32_t block_scan(uint32_t v, uint32_t* red, uint32_t* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint32_t incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  __syncthreads();
  if (lane == 63) red[w] = incl;
  __syncthreads();
  uint32_t before = 0, all = 0;
  for (int i = 0; i < T / 64; ++i) {
    before += i < w ? red[i] : 0u;
    all += red[i];
  }
  *total = all;
  return before + incl - v;
}

// Key of the n-th largest flagged key of the workgroup (at least n flagged):
// 8 bits per pass from the top, LDS histograms.
template <int T, int J>
__device__ uint32_t select_nth_key(const uint32_t (&key)[J], uint32_t flags, uint32_t n,
                                   uint32_t* hist, uint32_t* pick) {
  const int tid = threadIdx.x, lane = tid & 63;
  uint32_t prefix = 0, pmask = 0, need = n;
#pragma unroll 1
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int b = tid; b < 256; b += T) hist[b] = 0;
    __syncthreads();
    // Plain LDS atomics: they issue back to back (lanes on one address
    // serialize in the LDS unit, not in the wave).
#pragma unroll
    for (int j = 0; j < J; ++j)
      if ((flags >> j & 1u) && (key[j] & pmask) == prefix) atomicAdd(&hist[(key[j] >> shift) & 255u], 1u);
    __syncthreads();
    if (tid < 64) {
      // Lane L holds digits 255 - 4L .. 252 - 4L (the largest first).
      uint32_t c[4], t = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        c[q] = hist[255 - 4 * lane - q];
        t += c[q];
      }
      uint32_t incl = t;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = __shfl_up(incl, off, 64);
        if (lane >= off) incl += o;
      }
      uint32_t run = incl - t;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (run < need && run + c[q] >= need) {
          pick[0] = 255u - 4u * lane - q;
          pick[1] = run;
        }
        run += c[q];
      }
    }
    __syncthreads();
    need -= pick[1];
    prefix |= pick[0] << shift;
    pmask |= 255u << shift;
  }
  return prefix;
}

struct CandLayout {  // the workspace of one call
  float2* part;  // [beams][slices] (max, sum of exp)
  int* count;    // [beams][slices][2] entries kept per class
  float* x;      // [beams][slices][2][kc] logits
  int* token;    // [beams][slices][2][kc]
};
__host__ __device__ inline CandLayout cand_layout(void* ws, int beams, int slices, int kc) {
  char* p = static_cast<char*>(ws);
  CandLayout l;
  const int64_t parts = (int64_t)beams * slices;
  l.part = reinterpret_cast<float2*>(p);
  l.count = reinterpret_cast<int*>(p + parts * 8);
  l.x = reinterpret_cast<float*>(p + parts * 16);
  l.token = reinterpret_cast<int*>(p + parts * 16 + parts * 2 * kc * 4);
  return l;
}

__global__ __launch_bounds__(kSliceThreads) void cand_slice_kernel(BeamCandArgs a) {
  __shared__ float red[kSliceThreads / 64];
  __shared__ uint32_t ured[kSliceThreads / 64];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t pick[2];
  const int s = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  const int V = a.vocab, S = gridDim.x;
  const CandLayout l = cand_layout(a.workspace, a.beams, S, a.kc);
  const __amdgpu_buffer_rsrc_t lr = make_rsrc(a.logits + (int64_t)row * V, (uint32_t)V * 2u);
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.seen + (int64_t)row * a.seen_pitch, (uint32_t)V);
  float x[kSliceJ];
  uint32_t key[kSliceJ];
  uint32_t valid = 0, seen = 0;
#pragma unroll
  for (int j = 0; j < kSliceJ; ++j) {
    const uint32_t i = (uint32_t)(s * kSliceLen + j * kSliceThreads + tid);
    const uint32_t h = __builtin_amdgcn_raw_buffer_load_b16(lr, i * 2u, 0, 0);
    const uint32_t b = __builtin_amdgcn_raw_buffer_load_b8(sr, i, 0, 0);
    const bool ok = i < (uint32_t)V;
    x[j] = ok ? half_bits_to_float((uint16_t)h) : -INFINITY;
    valid |= (uint32_t)ok << j;
    seen |= (uint32_t)(ok && b != 0) << j;
  }
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < kSliceJ; ++j) m = fmaxf(m, x[j]);
  m = block_reduce<kSliceThreads>(m, true, red);
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < kSliceJ; ++j)
    if (valid >> j & 1u) sum += expf(x[j] - m);
  sum = block_reduce<kSliceThreads>(sum, false, red);
  if (tid == 0) l.part[row * S + s] = make_float2(m, sum);
#pragma unroll
  for (int j = 0; j < kSliceJ; ++j) key[j] = order_key(x[j]);

  for (int c = 0; c < 2; ++c) {  // 0: unseen tokens, 1: seen
    const uint32_t flags = valid & (c ? seen : ~seen);
    uint32_t cnt;
    block_scan<kSliceThreads>(__popc(flags), ured, &cnt);
    const uint32_t n = min(cnt, (uint32_t)a.kc);
    // The n-th largest key (every flagged key when there are at most kc).
    const uint32_t kth = cnt > (uint32_t)a.kc
                             ? select_nth_key<kSliceThreads, kSliceJ>(key, flags, n, hist, pick)
                             : 0u;
    uint32_t gt = 0, eq = 0;
#pragma unroll
    for (int j = 0; j < kSliceJ; ++j) {
      gt += (flags >> j & 1u) && key[j] > kth;
      eq += (flags >> j & 1u) && key[j] == kth;
    }
    uint32_t gtotal, etotal;
    uint32_t gslot = block_scan<kSliceThreads>(gt, ured, &gtotal);
    uint32_t eslot = gtotal + block_scan<kSliceThreads>(eq, ured, &etotal);
    const int64_t base = ((int64_t)(row * S + s) * 2 + c) * a.kc;
#pragma unroll
    for (int j = 0; j < kSliceJ; ++j) {
      if (!(flags >> j & 1u)) continue;
      uint32_t slot;
      if (key[j] > kth) slot = gslot++;
      else if (key[j] == kth) slot = eslot++;
      else continue;
      if (slot < n) {
        l.x[base + slot] = x[j];
        l.token[base + slot] = s * kSliceLen + j * kSliceThreads + tid;
      }
    }
    if (tid == 0) l.count[(row * S + s) * 2 + c] = (int)n;
  }
}

__global__ __launch_bounds__(kCandThreads) void cand_merge_kernel(BeamCandArgs a, int S) {
  __shared__ float red[kCandThreads / 64];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t pick[2];
  __shared__ int count;
  __shared__ float lv[kCandThreads * kMergeJ];
  __shared__ int li[kCandThreads * kMergeJ];
  __shared__ float sv[kCandMax];
  __shared__ int si[kCandMax];
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  __shared__ float row_lse[2];
  __shared__ int counts[2 * kMaxSlices];
  const CandLayout l = cand_layout(a.workspace, a.beams, S, a.kc);
  // The row's max and log of the sum of exp(x - max), from the slices (wave
  // 0, one slice per lane), and the slices' entry counts.
  if (tid < 64) {
    const float2 p = tid < S ? l.part[row * S + tid] : make_float2(-INFINITY, 0.f);
    float m = p.x;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    float sum = tid < S ? p.y * expf(p.x - m) : 0.f;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 64);
    if (tid == 0) {
      row_lse[0] = m;
      row_lse[1] = logf(sum);
    }
  } else if (tid < 64 + 2 * S) {
    counts[tid - 64] = l.count[row * S * 2 + tid - 64];
  }
  __syncthreads();
  const float m = row_lse[0], lse = row_lse[1];

  // Entry e: slice e / (2 kc), class (e / kc) % 2, slot e % kc.
  float v[kMergeJ];
  int tok[kMergeJ];
  uint32_t key[kMergeJ];
  uint32_t flags = 0;
#pragma unroll
  for (int j = 0; j < kMergeJ; ++j) {
    const int e = j * kCandThreads + tid;
    const int s = e / (2 * a.kc), c = (e / a.kc) % 2, slot = e % a.kc;
    const bool ok = s < S && slot < counts[s * 2 + c];
    float w = -INFINITY;
    tok[j] = 0;
    if (ok) {
      const int64_t at = ((int64_t)(row * S + s) * 2 + c) * a.kc + slot;
      const float lp = (l.x[at] - m) - lse;
      w = c == 0 ? lp : lp < 0.f ? lp * a.penalty : lp / a.penalty;
      tok[j] = l.token[at];
    }
    key[j] = order_key(w);
    v[j] = a.temperature != 1.0f ? w / a.temperature : w;
    flags |= (uint32_t)ok << j;
  }
  const uint32_t kth = select_nth_key<kCandThreads, kMergeJ>(key, flags, (uint32_t)a.kc, hist, pick);

  // Every entry with w >= the kc-th largest, sorted: v descending, token
  // ascending.
  if (tid == 0) count = 0;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kMergeJ; ++j) {
    const bool ok = (flags >> j & 1u) && key[j] >= kth;
    const uint64_t mask = __ballot(ok);
    if (mask) {
      const int leader = __ffsll((unsigned long long)mask) - 1;
      int base = 0;
      if (lane == leader) base = atomicAdd(&count, __popcll(mask));
      base = __builtin_amdgcn_readlane(base, leader);
      const int slot = base + (int)__builtin_amdgcn_mbcnt_hi(
                                  (uint32_t)(mask >> 32),
                                  __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
      if (ok) {
        lv[slot] = v[j];
        li[slot] = tok[j];
      }
    }
  }
  __syncthreads();
  const int n = count;
  for (int t = tid; t < n; t += kCandThreads) {
    const float x = lv[t];
    const int ix = li[t];
    int rank = 0;
    for (int u = 0; u < n; ++u) rank += lv[u] > x || (lv[u] == x && li[u] < ix);
    if (rank < a.kc) {
      sv[rank] = x;
      si[rank] = ix;
    }
  }
  __syncthreads();

  if (tid < 64) {
    const int d = lane;
    const bool in = d < a.kc;
    float x = in ? sv[d] : -INFINITY;
    const float thr = sv[a.k - 1];
    const bool overflow = a.kc < a.vocab && sv[a.kc - 1] == thr;
    if (x < thr) x = -INFINITY;
    if (a.use_top_p) {
      const float mx = sv[0];
      const float e = x == -INFINITY ? 0.f : expf(x - mx);
      float s = e;
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
      const float p = e / s;
      // Sum of p over this entry and every smaller one (d' >= d).
      float acc = p;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float o = __shfl_down(acc, off, 64);
        if (d + off < 64) acc += o;
      }
      if (acc <= a.top_p_cut && d >= a.keep) x = -INFINITY;
    }
    if (in) {
      a.candidates[(int64_t)row * a.kc + d] = si[d];
      a.scores[(int64_t)row * a.kc + d] = x + a.running[row];
    }
    if (d == 0) a.status[2 + row] = overflow;
  }
}

__global__ __launch_bounds__(kCandThreads) void beam_joint_kernel(BeamCandArgs a) {
  __shared__ float red[kCandThreads / 64];
  __shared__ int nonzero, nans;
  const int tid = threadIdx.x;
  const int n = a.beams * a.kc;
  const float s = tid < n ? a.scores[tid] : -INFINITY;
  const float m = block_reduce<kCandThreads>(s, true, red);
  const float e = s == -INFINITY ? 0.f : expf(s - m);
  const float total = block_reduce<kCandThreads>(e, false, red);
  const float p = e / total;
  if (tid == 0) nonzero = 0, nans = 0;
  __syncthreads();
  // Possible draws: probabilities > 0 (a NaN counts as none). A NaN
  // probability makes the count -1: torch.multinomial rejects such input,
  // and the caller raises its error instead of drawing.
  const uint64_t mask = __ballot(tid < n && p > 0.f);
  const uint64_t nan_mask = __ballot(tid < n && p != p);
  if ((tid & 63) == 0 && mask) atomicAdd(&nonzero, __popcll(mask));
  if ((tid & 63) == 0 && nan_mask) atomicAdd(&nans, 1);
  if (tid < n) a.probs[tid] = p;
  __syncthreads();
  if (tid == 0) {
    int64_t any = 0;
    for (int r = 0; r < a.beams; ++r) any |= a.status[2 + r];
    a.status[0] = nans ? -1 : nonzero;
    a.status[1] = any;
  }
}

}  // namespace

int beam_candidate_slices(int vocab) { return (vocab + kSliceLen - 1) / kSliceLen; }

int64_t beam_candidates_workspace(int beams, int vocab, int kc) {
  const int64_t parts = (int64_t)beams * beam_candidate_slices(vocab);
  return parts * 16 + parts * 2 * kc * 8;
}

hipError_t launch_beam_candidates(const BeamCandArgs& a, hipStream_t stream) {
  const int S = beam_candidate_slices(a.vocab);
  hipLaunchKernelGGL(cand_slice_kernel, dim3(S, a.beams), dim3(kSliceThreads), 0, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(cand_merge_kernel, dim3(a.beams), dim3(kCandThreads), 0, stream, a, S);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(beam_joint_kernel, dim3(1), dim3(kCandThreads), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_beam_select(const BeamSelectArgs& a, hipStream_t stream) {
  const int64_t pieces = a.beams * (a.seen_pitch / 16);
  const int64_t per_block = (int64_t)kThreads * kSeenPieces;
  const int blocks = (int)((pieces + per_block - 1) / per_block);
  hipLaunchKernelGGL(beam_select_kernel, dim3(blocks < 1 ? 1 : blocks), dim3(kThreads), 0,
                     stream, a);
  return hipGetLastError();
}

}  // namespace svq
