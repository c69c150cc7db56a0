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
    qv[e] = a.probs[f] / a.noise[f];
  }
  __syncthreads();

  // Wave 0: `draws` rounds of the race's maximum over the entries not yet
  // drawn; lane l owns entries l, l + 64, ... (held in registers).
  __shared__ int64_t dpick[kMaxDraws];
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
#pragma unroll
      for (int i = 0; i < kPerLane; ++i)
        if (!(taken >> i & 1u) && ahead(q[i], f[i], bq, bf)) {
          bq = q[i];
          bf = f[i];
        }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        const float oq = __shfl_xor(bq, off, 64);
        const int64_t of = __shfl_xor(bf, off, 64);
        if (ahead(oq, of, bq, bf)) {
          bq = oq;
          bf = of;
        }
      }
      // Every lane holds the winner; its owner marks it drawn.
#pragma unroll
      for (int i = 0; i < kPerLane; ++i) taken |= (uint32_t)(f[i] == bf) << i;
      if (lane == 0) dpick[d] = bf;
    }
  }
  __syncthreads();
  if (tid < a.draws) dscore[tid] = a.scores[dpick[tid]];
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

}  // namespace

hipError_t launch_beam_select(const BeamSelectArgs& a, hipStream_t stream) {
  const int64_t pieces = a.beams * (a.seen_pitch / 16);
  const int64_t per_block = (int64_t)kThreads * kSeenPieces;
  const int blocks = (int)((pieces + per_block - 1) / per_block);
  hipLaunchKernelGGL(beam_select_kernel, dim3(blocks < 1 ? 1 : blocks), dim3(kThreads), 0,
                     stream, a);
  return hipGetLastError();
}

}  // namespace svq
