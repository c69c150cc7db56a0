// Fused GGUF SoA dequantize + GEMV on the gfx950 matrix cores
// (v_mfma_f32_16x16x32_f16), for 1 <= M <= 8 activation rows.
//
// Same arithmetic as the reference `_soa_gemv` (quantization.py:171-229): a
// 32-weight block's integer-code dot product is formed in fp32 and multiplied
// by the block's fp16 scale once; bias is added in fp32; fp16 or fp32 out.
//
// One MFMA is one block of 16 weight rows:
//   D[m][n] = sum_{k < 32} x[m][32b + kmap(k)] * code[n][32b + kmap(k)] + C[m][n]
// with A = the activations (16 rows; rows >= M repeat real rows and are
// ignored), B = the 16 rows' codes placed directly as fp16 subnormals (exact
// products), C = -offset * sum_k x[m][32b + k] (removes the code offset), and
// the fp32 result scaled by the block's scale into the row accumulators. A
// lane (n16 = lane % 16, t = lane / 16) supplies B's 8 k-slots of weight row
// n16, which are the block's weights 4t..4t+3 and 16+4t..16+4t+3: exactly
// the low and high nibbles of payload bytes 4t..4t+3 (Q4_0/Q5_0), or int8
// bytes 4t..4t+3 and 16+4t..16+4t+3 (Q8_0). x is staged in LDS permuted the
// same way.
//
// Loads: each lane reads 16 contiguous payload bytes of its row per step (a
// whole Q4_0 block, a Q5_0 block as 4 + 16 bytes, or half a Q8_0 block), so
// the 4 lanes of a row read 64-80 contiguous bytes. A 4 x 4 transpose across
// the lane groups t (v_permlane32_swap + v_permlane16_swap) then gives every
// lane its dword t of each of the step's blocks.
//
// Work split: a workgroup of P x S waves; wave (p, s) owns row tile p of each
// tile group the workgroup processes and the step range s of K. Workgroups
// are persistent over tile groups. With S > 1 the S partial sums of a tile
// are added through LDS at the end of each tile group. Each wave keeps a
// ring of D steps of payload in flight across tile boundaries; loads past
// the end use an out-of-range buffer offset (zeros, no memory access).
#include "svq_device.h"
#include "svq_launch.h"

namespace svq {

namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr uint32_t kOutOfRange = 0x80000000u;  // past every buffer range (< 2^31 bytes)

// Per-qtype geometry. Codes go into B as fp16 subnormals: 16 * code (Q4_0,
// Q5_0: code < 32, so at most 496 * 2^-24) or int8 + 128 (Q8_0).
template <int QT> struct MfmaTraits;
template <> struct MfmaTraits<4> {
  static constexpr int kBlocksPerStep = 4;
  static constexpr int kBlockBytes = 16;
  static constexpr int kScaleDwords = 2;
  static constexpr float kCScale = -0x1p-17f;  // -8 * 16 * 2^-24
  static constexpr float kOutScale = 0x1p20f;
};
template <> struct MfmaTraits<5> {
  static constexpr int kBlocksPerStep = 4;
  static constexpr int kBlockBytes = 20;
  static constexpr int kScaleDwords = 2;
  static constexpr float kCScale = -0x1p-16f;  // -16 * 16 * 2^-24
  static constexpr float kOutScale = 0x1p20f;
};
template <> struct MfmaTraits<8> {
  static constexpr int kBlocksPerStep = 2;
  static constexpr int kBlockBytes = 32;
  static constexpr int kScaleDwords = 1;
  static constexpr float kCScale = -0x1p-17f;  // -128 * 2^-24
  static constexpr float kOutScale = 0x1p24f;
};

// Transpose 4 x 4 dwords across the lane groups t = lane / 16: on entry lane
// group t holds v[0..3] of source t; on exit lane group t holds dword t of
// every source j in v[j].
__device__ __forceinline__ void transpose4(uint32_t (&v)[4]) {
  auto s = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
  v[0] = s[0]; v[2] = s[1];
  s = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
  v[1] = s[0]; v[3] = s[1];
  s = __builtin_amdgcn_permlane16_swap(v[0], v[1], false, false);
  v[0] = s[0]; v[1] = s[1];
  s = __builtin_amdgcn_permlane16_swap(v[2], v[3], false, false);
  v[2] = s[0]; v[3] = s[1];
}

// B operand of one block for lane group t: k-slots 0-3 = weights 4t..4t+3,
// 4-7 = weights 16+4t..16+4t+3.
__device__ __forceinline__ h8_t codes_q4(uint32_t w) {
  const uint32_t lo = (w << 4) & 0xf0f0f0f0u;  // 16 * low nibbles
  const uint32_t hi = w & 0xf0f0f0f0u;         // 16 * high nibbles
  u32x4 p;
  p.x = perm(0u, lo, kSelB01);
  p.y = perm(0u, lo, kSelB23);
  p.z = perm(0u, hi, kSelB01);
  p.w = perm(0u, hi, kSelB23);
  return __builtin_bit_cast(h8_t, p);
}

// Q5_0: nibble dword w (payload bytes 4t..4t+3) and the block's mask qh;
// the fifth bit becomes the high byte of each half: 16 * nibble + 256 * bit.
__device__ __forceinline__ h8_t codes_q5(uint32_t w, uint32_t qh, uint32_t t4) {
  const uint32_t lo = (w << 4) & 0xf0f0f0f0u;
  const uint32_t hi = w & 0xf0f0f0f0u;
  const uint32_t blo = spread4(__builtin_amdgcn_ubfe(qh, t4, 4));
  const uint32_t bhi = spread4(__builtin_amdgcn_ubfe(qh, t4 + 16u, 4));
  u32x4 p;
  p.x = perm(blo, lo, kSelB01H);
  p.y = perm(blo, lo, kSelB23H);
  p.z = perm(bhi, hi, kSelB01H);
  p.w = perm(bhi, hi, kSelB23H);
  return __builtin_bit_cast(h8_t, p);
}

// Q8_0: int8 bytes 4t..4t+3 (w0) and 16+4t..16+4t+3 (w1) as int8 + 128.
__device__ __forceinline__ h8_t codes_q8(uint32_t w0, uint32_t w1) {
  const uint32_t a = w0 ^ 0x80808080u, b = w1 ^ 0x80808080u;
  u32x4 p;
  p.x = perm(0u, a, kSelB01);
  p.y = perm(0u, a, kSelB23);
  p.z = perm(0u, b, kSelB01);
  p.w = perm(0u, b, kSelB23);
  return __builtin_bit_cast(h8_t, p);
}

// Stage x into LDS as the A operand: entry (b, t, m) (16 bytes, at index
// (b * 4 + t) * M + m) holds x[m][32b + 4t + 0..3] and x[m][32b + 16 + 4t + 0..3].
// cs[b * MC + m] = kCScale * sum_k x[m][32b + k] (zero for M <= m < MC).
template <int QT, int M, int MC>
__device__ __forceinline__ void stage_x_mfma(const uint16_t* __restrict__ x, int k, u32x4* xa,
                                             float* cs, int tid, int nthreads) {
  constexpr int NB = 4;  // items per thread per batch: loads first, then LDS writes
  const int kb = k >> 5;
  const int items = kb * MC;
  const uint32_t ones = 0x3c003c00u;  // fp16 (1, 1)
  for (int base = 0; base < items; base += NB * nthreads) {
    u32x4 v[NB][4];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int it = base + i * nthreads + tid;
      const int b = it / MC, m = it % MC;
      if (it < items && m < M) {
        const u32x4* src = reinterpret_cast<const u32x4*>(x + (size_t)m * k + 32 * b);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[i][j] = src[j];
      }
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int it = base + i * nthreads + tid;
      const int b = it / MC, m = it % MC;
      if (it >= items) continue;
      if (m >= M) {
        cs[it] = 0.f;
        continue;
      }
      uint32_t u[16];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u[4 * j] = v[i][j].x; u[4 * j + 1] = v[i][j].y;
        u[4 * j + 2] = v[i][j].z; u[4 * j + 3] = v[i][j].w;
      }
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        u32x4 e;
        e.x = u[2 * tt]; e.y = u[2 * tt + 1];
        e.z = u[8 + 2 * tt]; e.w = u[9 + 2 * tt];
        xa[(b * 4 + tt) * M + m] = e;
      }
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) s0 = dot2(u[j], ones, s0);
#pragma unroll
      for (int j = 8; j < 16; ++j) s1 = dot2(u[j], ones, s1);
      cs[it] = (s0 + s1) * MfmaTraits<QT>::kCScale;
    }
  }
}

template <int QT, int M, int R, int D, int B>
__global__ __launch_bounds__(1024) void gemv_mfma_kernel(GemvArgs a) {
  static_assert(D % B == 0, "ring refills in bursts of B slots");
  using T = MfmaTraits<QT>;
  constexpr int BPS = T::kBlocksPerStep;
  constexpr int MC = (M + 3) / 4 * 4;       // offset-sum rows per block
  constexpr int MI = M < 4 ? M : 4;         // accumulator rows per lane
  extern __shared__ u32x4 lds[];

  const int n = a.n, k = a.k;
  const int kb = k >> 5;
  const int steps = kb / BPS;
  const int S = a.ksplit, P = a.slots;
  const int W = P * S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int s_id = wave % S, p_id = wave / S;
  const int n16 = lane & 15, t = lane >> 4;
  const int s0 = s_id * steps / S, s1 = (s_id + 1) * steps / S;
  const int my_steps = s1 - s0;
  const int tile_rows = 16 * R;
  const int tiles = (n + tile_rows - 1) / tile_rows;
  const int groups = (tiles + P - 1) / P;
  const int G = gridDim.x;
  const int my_groups = (int)blockIdx.x < groups ? (groups - (int)blockIdx.x + G - 1) / G : 0;
  const int total = my_groups * my_steps;
  const uint32_t row_bytes = (uint32_t)kb * T::kBlockBytes;

  const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q, (uint32_t)n * row_bytes);
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.s, (uint32_t)n * (uint32_t)kb * 2u);
  const __amdgpu_buffer_rsrc_t br = make_rsrc(a.bias, a.bias ? (uint32_t)n * 2u : 0u);

  u32x4* xa = lds;
  float* cs = reinterpret_cast<float*>(lds + kb * 4 * M);
  f4_t* part = reinterpret_cast<f4_t*>(cs + kb * MC);  // [2][W][R][64] partial sums

  // Stage x before any weight load (vector loads retire in order: x loads
  // behind the weight prologue would wait for all of it).
  stage_x_mfma<QT, M, MC>(a.x, k, xa, cs, threadIdx.x, W * 64);
  __syncthreads();

  // Row offsets of this lane's R rows in tile group ordinal j; a row past n
  // gets an out-of-range offset.
  auto row_offsets = [&](int j, uint32_t (&qo)[R], uint32_t (&so)[R]) {
    const int tile = ((int)blockIdx.x + j * G) * P + p_id;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = tile * tile_rows + r * 16 + n16;
      const bool ok = j < my_groups && row < n;
      const uint32_t oob = (uint32_t)(!ok) * kOutOfRange;
      const uint32_t rr = ok ? (uint32_t)row : 0u;
      qo[r] = rr * row_bytes + oob;
      so[r] = rr * (uint32_t)kb * 2u + oob;
    }
  };

  // Ring of D steps: payload dwords, Q5_0 mask, scale dwords, per row tile.
  uint32_t wq[D][R][4];
  uint32_t wh[D][R];
  uint32_t ws[D][R][T::kScaleDwords];
  int pj = 0, ps = s0;
  uint32_t pqo[R], pso[R];
  row_offsets(0, pqo, pso);
  // Lane part of the payload offset within a step.
  const uint32_t lane_q = QT == 8 ? (uint32_t)t * 16u : (uint32_t)t * T::kBlockBytes;
  auto issue = [&](int d) {
    // A finished wave keeps loading its last (out-of-range) offsets: zeros.
    const uint32_t qstep = (uint32_t)ps * (BPS * T::kBlockBytes) + lane_q;
    const uint32_t sstep = (uint32_t)ps * (BPS * 2);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if constexpr (QT == 5) {
        wh[d][r] = __builtin_amdgcn_raw_buffer_load_b32(qr, pqo[r] + qstep, 0, 0);
        const u32x4 v = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, pqo[r] + qstep + 4u, 0, 0));
        wq[d][r][0] = v.x; wq[d][r][1] = v.y; wq[d][r][2] = v.z; wq[d][r][3] = v.w;
      } else {
        const u32x4 v = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, pqo[r] + qstep, 0, 0));
        wq[d][r][0] = v.x; wq[d][r][1] = v.y; wq[d][r][2] = v.z; wq[d][r][3] = v.w;
      }
      if constexpr (T::kScaleDwords == 2) {
        const u32x2 v = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_raw_buffer_load_b64(sr, pso[r] + sstep, 0, 0));
        ws[d][r][0] = v.x; ws[d][r][1] = v.y;
      } else {
        ws[d][r][0] = __builtin_amdgcn_raw_buffer_load_b32(sr, pso[r] + sstep, 0, 0);
      }
    }
    if (++ps == s1) {
      ps = s0;
      ++pj;
      row_offsets(pj, pqo, pso);
    }
  };

  auto load_bias = [&](int j, uint32_t (&bb)[R]) {
    const int tile = ((int)blockIdx.x + j * G) * P + p_id;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = tile * tile_rows + r * 16 + n16;
      const uint32_t oob = (uint32_t)(!(j < my_groups && row < n)) * kOutOfRange;
      bb[r] = __builtin_amdgcn_raw_buffer_load_b16(br, (uint32_t)(row < n ? row : 0) * 2u + oob,
                                                   0, 0);
    }
  };

#pragma unroll
  for (int d = 0; d < D; ++d) issue(d);
  uint32_t bias_bits[R];
  load_bias(0, bias_bits);

  f4_t acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = f4_t{0.f, 0.f, 0.f, 0.f};

  // LDS addresses of this lane's A entries (row n16 % M, lane group t) and C
  // values (rows 4t..4t+3, clamped to the staged MC rows).
  const int a_lane = t * M + n16 % M;
  const int c_lane = 4 * (t < MC / 4 ? t : MC / 4 - 1);
  const uint32_t t4 = 4u * (uint32_t)t;

  int cj = 0, cs_ = s0;  // tile group ordinal and step of the current ring slot
  for (int it = 0; it < total; it += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      if (it + d < total) {
        uint32_t q[R][4];
        uint32_t qh[R][4];
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
          for (int i = 0; i < 4; ++i) q[r][i] = wq[d][r][i];
          transpose4(q[r]);
          if constexpr (QT == 5) {
#pragma unroll
            for (int i = 0; i < 4; ++i) qh[r][i] = wh[d][r];
            transpose4(qh[r]);
          }
        }
#pragma unroll
        for (int j = 0; j < BPS; ++j) {
          const int b = cs_ * BPS + j;
          const h8_t av = __builtin_bit_cast(h8_t, xa[b * 4 * M + a_lane]);
          const f4_t cv = *reinterpret_cast<const f4_t*>(cs + b * MC + c_lane);
#pragma unroll
          for (int r = 0; r < R; ++r) {
            h8_t bv;
            if constexpr (QT == 4) bv = codes_q4(q[r][j]);
            else if constexpr (QT == 5) bv = codes_q5(q[r][j], qh[r][j], t4);
            else bv = codes_q8(q[r][2 * j], q[r][2 * j + 1]);
            const f4_t dv = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, cv, 0, 0, 0);
            const float scale = half_bits_to_float(
                (uint16_t)(ws[d][r][j >> 1] >> (16 * (j & 1))));
#pragma unroll
            for (int i = 0; i < MI; ++i) acc[r][i] = __builtin_fmaf(dv[i], scale, acc[r][i]);
          }
        }
      }
      // Refill in bursts of B consecutive steps, so that each row's loads
      // reach the memory controllers as runs of B * 64 (80) contiguous bytes.
      if (d % B == B - 1) {
#pragma unroll
        for (int e = d - B + 1; e <= d; ++e) issue(e);
      }
      if (it + d < total && ++cs_ == s1) {
        // End of this wave's share of the tile group.
        const int tile = ((int)blockIdx.x + cj * G) * P + p_id;
        if (S > 1) {
          f4_t* buf = part + (size_t)((cj & 1) * W) * R * 64;
#pragma unroll
          for (int r = 0; r < R; ++r) buf[(wave * R + r) * 64 + lane] = acc[r];
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
          __builtin_amdgcn_s_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
          if (s_id == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
              f4_t v = buf[((p_id * S) * R + r) * 64 + lane];
              for (int o = 1; o < S; ++o) v += buf[((p_id * S + o) * R + r) * 64 + lane];
              acc[r] = v;
            }
          }
        }
        if (s_id == 0) {
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const int row = tile * tile_rows + r * 16 + n16;
            if (row < n) {
              const float bsum = half_bits_to_float((uint16_t)bias_bits[r]);
#pragma unroll
              for (int i = 0; i < MI; ++i) {
                const int m = 4 * t + i;
                if (m < M) {
                  const float v = __builtin_fmaf(acc[r][i], T::kOutScale, bsum);
                  store_y(a, m, row, v);
                }
              }
            }
          }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = f4_t{0.f, 0.f, 0.f, 0.f};
        cs_ = s0;
        ++cj;
        load_bias(cj, bias_bits);
      }
    }
  }
}

template <int QT, int M, int R, int D, int B>
const void* mfma_kernel_ptr() {
  return reinterpret_cast<const void*>(&gemv_mfma_kernel<QT, M, R, D, B>);
}

template <int QT, int M, int R, int D, int B>
hipError_t mfma_launch(const GemvArgs& a, int groups, int wpg, size_t lds, hipStream_t stream) {
  hipLaunchKernelGGL((gemv_mfma_kernel<QT, M, R, D, B>), dim3(groups), dim3(wpg * 64), lds,
                     stream, a);
  return hipGetLastError();
}

// (R, D, B): one 16-row tile per wave with an 8-step ring refilled 4 steps at
// a time, or two tiles (sharing each A and C read) with a 4-step ring
// refilled 2 at a time.
template <int QT, int M>
hipError_t mfma_dispatch_r(const GemvArgs& a, int rows, int groups, int wpg, size_t lds,
                           hipStream_t stream, const void** fn) {
  if (rows == 2) {
    if (fn) { *fn = mfma_kernel_ptr<QT, M, 2, 4, 2>(); return hipSuccess; }
    return mfma_launch<QT, M, 2, 4, 2>(a, groups, wpg, lds, stream);
  }
  if (fn) { *fn = mfma_kernel_ptr<QT, M, 1, 8, 4>(); return hipSuccess; }
  return mfma_launch<QT, M, 1, 8, 4>(a, groups, wpg, lds, stream);
}

template <int QT>
hipError_t mfma_dispatch_m(const GemvArgs& a, int m, int rows, int groups, int wpg, size_t lds,
                           hipStream_t stream, const void** fn) {
  switch (m) {
    case 1: return mfma_dispatch_r<QT, 1>(a, rows, groups, wpg, lds, stream, fn);
    case 2: return mfma_dispatch_r<QT, 2>(a, rows, groups, wpg, lds, stream, fn);
    case 3: return mfma_dispatch_r<QT, 3>(a, rows, groups, wpg, lds, stream, fn);
    case 4: return mfma_dispatch_r<QT, 4>(a, rows, groups, wpg, lds, stream, fn);
    case 5: return mfma_dispatch_r<QT, 5>(a, rows, groups, wpg, lds, stream, fn);
    case 6: return mfma_dispatch_r<QT, 6>(a, rows, groups, wpg, lds, stream, fn);
    case 7: return mfma_dispatch_r<QT, 7>(a, rows, groups, wpg, lds, stream, fn);
    case 8: return mfma_dispatch_r<QT, 8>(a, rows, groups, wpg, lds, stream, fn);
  }
  return hipErrorInvalidValue;
}

hipError_t mfma_dispatch(const GemvArgs& a, int qtype, int m, int rows, int groups, int wpg,
                         size_t lds, hipStream_t stream, const void** fn) {
  switch (qtype) {
    case 4: return mfma_dispatch_m<4>(a, m, rows, groups, wpg, lds, stream, fn);
    case 5: return mfma_dispatch_m<5>(a, m, rows, groups, wpg, lds, stream, fn);
    case 8: return mfma_dispatch_m<8>(a, m, rows, groups, wpg, lds, stream, fn);
  }
  return hipErrorInvalidValue;
}

}  // namespace

int mfma_blocks_per_step(int qtype) { return qtype == 8 ? 2 : 4; }

size_t mfma_lds_bytes(int qtype, int m, int k, int rows, int wpg, int ksplit) {
  (void)qtype;
  const size_t kb = (size_t)(k / 32);
  const size_t mc = (size_t)(m + 3) / 4 * 4;
  size_t bytes = kb * 4 * m * 16 + kb * mc * 4;
  if (ksplit > 1) bytes += (size_t)2 * wpg * rows * 64 * 16;
  return bytes;
}

const void* mfma_kernel(int qtype, int m, int rows) {
  const void* fn = nullptr;
  GemvArgs unused{};
  (void)mfma_dispatch(unused, qtype, m, rows, 0, 0, 0, nullptr, &fn);
  return fn;
}

hipError_t launch_gemv_mfma(const GemvArgs& a, int qtype, int m, int rows, int groups,
                            hipStream_t stream) {
  const int wpg = a.slots * a.ksplit;
  return mfma_dispatch(a, qtype, m, rows, groups, wpg,
                       mfma_lds_bytes(qtype, m, a.k, rows, wpg, a.ksplit), stream, nullptr);
}

}  // namespace svq
