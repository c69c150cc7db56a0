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
    qv[e] = a.probs[a.compact ? e : f] / a.noise[f];
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
// warped log-probabilities instead of the whole vocabulary. Kernel 1 (one
// workgroup per beam row) keeps the row's fp16 logits in registers (64 per
// thread) and forms
//   log_softmax(x) = (x - max) - log(sum exp(x - max))  (expf / logf);
//   w = penalty: seen ? (lp < 0 ? lp * p : lp / p) : lp;  v = w / t
//   (temperature t; no division at t = 1).
// The kc largest are found on w (v is monotone in w, so the order agrees;
// ties that the division creates at the kc-th value only matter where that
// value is also the k-th, which is reported as overflow): a 4-pass radix
// select on order-preserving keys (wave-aggregated LDS histograms), then
// every entry at or above the kc-th largest is sorted on v (descending,
// token ascending). Top-k: values below the k-th largest become -inf. Top-p
// over the kc values: softmax, sums from the smallest up, removal where the
// sum <= 1 - top_p except the `keep` largest. Candidate score = v +
// running[row]. Kernel 2 (one workgroup) makes the joint softmax over all
// candidates, the number of non-zero probabilities and the overflow flag.
// The sums add in another order than torch's reductions (the results agree
// to rounding); comparisons, the penalty, the temperature and the score
// additions are the same fp32 operations.
constexpr int kCandThreads = 1024;
constexpr int kCandPerThread = kCandMaxVocab / kCandThreads;  // 64, as fp16 pairs
constexpr int kCandCap = 1024;  // entries >= the kc-th largest kept for the sort
constexpr int kCandWaves = kCandThreads / 64;

__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t b = __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Block-wide max / sum over kCandThreads threads, the same order every call.
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
  for (int i = 1; i < kCandWaves; ++i) r = is_max ? fmaxf(r, red[i]) : r + red[i];
  return r;
}

__global__ __launch_bounds__(kCandThreads) void beam_candidates_kernel(BeamCandArgs a) {
  __shared__ float red[kCandWaves];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t pick[2];  // digit, entries above it
  __shared__ int count;
  __shared__ float lv[kCandCap];
  __shared__ int li[kCandCap];
  __shared__ float sv[kCandMax];
  __shared__ int si[kCandMax];
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  const int V = a.vocab;
  // Buffer loads of the row (32-bit offsets; reads past it return 0).
  const __amdgpu_buffer_rsrc_t lr = make_rsrc(a.logits + (int64_t)row * V, (uint32_t)V * 2u);
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.seen + (int64_t)row * a.seen_pitch, (uint32_t)V);

  // Element j of this thread: token j * kCandThreads + tid; fp16 bits, two
  // per register (past the vocabulary: -inf, never counted).
  uint32_t xh[kCandPerThread / 2];
  uint64_t seen_bits = 0;
#pragma unroll
  for (int j = 0; j < kCandPerThread; j += 2) {
    const uint32_t i0 = (uint32_t)(j * kCandThreads + tid), i1 = i0 + kCandThreads;
    uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(lr, i0 * 2u, 0, 0);
    uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(lr, i1 * 2u, 0, 0);
    lo = i0 < (uint32_t)V ? lo : 0xfc00u;
    hi = i1 < (uint32_t)V ? hi : 0xfc00u;
    xh[j / 2] = lo | hi << 16;
    seen_bits |= (uint64_t)(__builtin_amdgcn_raw_buffer_load_b8(sr, i0, 0, 0) != 0) << j;
    seen_bits |= (uint64_t)(__builtin_amdgcn_raw_buffer_load_b8(sr, i1, 0, 0) != 0) << (j + 1);
    if (j % 32 == 30) asm volatile("" ::: "memory");  // at most 64 loads in flight
  }
  auto x_of = [&](int j) {
    return half_bits_to_float((uint16_t)(j & 1 ? xh[j / 2] >> 16 : xh[j / 2] & 0xffffu));
  };
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < kCandPerThread; ++j) m = fmaxf(m, x_of(j));
  m = block_reduce(m, true, red);
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < kCandPerThread; ++j)
    if (j * kCandThreads + tid < V) sum += expf(x_of(j) - m);
  sum = block_reduce(sum, false, red);
  const float lse = logf(sum);
  // The penalized log-probability w of each element (v = w / temperature),
  // held as its order-preserving key; 0 (below every finite value's key)
  // past the vocabulary.
  uint32_t kv[kCandPerThread];
#pragma unroll
  for (int j = 0; j < kCandPerThread; ++j) {
    const float lp = (x_of(j) - m) - lse;
    const float w = !(seen_bits >> j & 1u) ? lp : lp < 0.f ? lp * a.penalty : lp / a.penalty;
    kv[j] = j * kCandThreads + tid < V ? order_key(w) : 0u;
  }

  // Radix select of the kc-th largest w, 8 bits per pass from the top.
  uint32_t prefix = 0, pmask = 0;
  uint32_t need = (uint32_t)a.kc;
#pragma unroll 1
  for (int shift = 24; shift >= 0; shift -= 8) {
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kCandPerThread; ++j) {
      const uint32_t key = kv[j];
      const bool ok = key != 0u && (key & pmask) == prefix;
      const uint32_t digit = (key >> shift) & 255u;
      // Lanes that share a digit add once (up to 4 digits per wave; the
      // rest add one each): few distinct digits mean many equal addresses.
      uint64_t act = __ballot(ok);
      for (int r = 0; r < 4 && act; ++r) {
        const int leader = __ffsll((unsigned long long)act) - 1;
        const uint32_t d0 = __shfl(digit, leader, 64);
        const uint64_t same = __ballot((act >> lane & 1u) && digit == d0);
        if (lane == leader) atomicAdd(&hist[d0], (uint32_t)__popcll(same));
        act &= ~same;
      }
      if (act >> lane & 1u) atomicAdd(&hist[digit], 1u);
    }
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
  const uint32_t kth = prefix;  // key of the kc-th largest w

  // Every entry with w >= the kc-th largest, as (v, token); then sorted: v
  // descending, token ascending.
  if (tid == 0) count = 0;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kCandPerThread; ++j) {
    const int i = j * kCandThreads + tid;
    const bool ok = kv[j] != 0u && kv[j] >= kth;
    const uint64_t mask = __ballot(ok);
    if (mask) {
      const int leader = __ffsll((unsigned long long)mask) - 1;
      int base = 0;
      if (lane == leader) base = atomicAdd(&count, __popcll(mask));
      base = __shfl(base, leader, 64);
      const int slot = base + (int)__builtin_amdgcn_mbcnt_hi(
                                  (uint32_t)(mask >> 32),
                                  __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
      if (ok && slot < kCandCap) {
        const float w = key_value(kv[j]);
        lv[slot] = a.temperature != 1.0f ? w / a.temperature : w;
        li[slot] = i;
      }
    }
  }
  __syncthreads();
  const int total = count;
  const int n = min(total, kCandCap);
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
    const bool overflow = total > kCandCap || (a.kc < V && sv[a.kc - 1] == thr);
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
  __shared__ float red[kCandWaves];
  __shared__ int nonzero;
  const int tid = threadIdx.x;
  const int n = a.beams * a.kc;
  const float s = tid < n ? a.scores[tid] : -INFINITY;
  const float m = block_reduce(s, true, red);
  const float e = s == -INFINITY ? 0.f : expf(s - m);
  const float total = block_reduce(e, false, red);
  const float p = e / total;
  if (tid == 0) nonzero = 0;
  __syncthreads();
  const uint64_t mask = __ballot(tid < n && p != 0.f);
  if ((tid & 63) == 0 && mask) atomicAdd(&nonzero, __popcll(mask));
  if (tid < n) a.probs[tid] = p;
  __syncthreads();
  if (tid == 0) {
    int64_t any = 0;
    for (int r = 0; r < a.beams; ++r) any |= a.status[2 + r];
    a.status[0] = nonzero;
    a.status[1] = any;
  }
}

}  // namespace

hipError_t launch_beam_candidates(const BeamCandArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(beam_candidates_kernel, dim3(a.beams), dim3(kCandThreads), 0, stream, a);
  hipError_t e = hipGetLastError();
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
