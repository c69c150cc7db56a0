// Fused GGUF SoA dequantize + GEMV for gfx950: y[m, n] = sum_k x[m,k] W[n,k]
// + bias[n] for 1 <= M <= 8, Q4_0 / Q5_0 / Q8_0. Replaces the reference's
// `_soa_gemv` Triton kernel (quantization.py:171-229) and, for beams 3..8,
// `_soa_mm` (quantization.py:130-169).
//
// Work mapping (one workgroup = 4 wave64s):
//   * A row of the weight matrix is split into units (svq_device.h). G lanes
//     (a power of two <= 64) cooperate on a row and stride over its units, so
//     each load instruction of a lane group reads G * 16 (or 20) contiguous
//     bytes. A wave holds 64 / G such row groups, each owning R consecutive
//     rows that reuse the activations held in registers.
//   * The activations x[M, K] are staged once per workgroup into LDS, in
//     "piece-major" order (16-byte piece p of unit u of row m at
//     [(m * P + p) * chunk + u]) so that lanes reading consecutive units read
//     consecutive 16-byte LDS words. Long K is staged in chunks that fit the
//     LDS budget. While staging, the workgroup also stores for every unit and
//     activation row offset * sum(x over the unit), the term that removes the
//     code offset (-8, -16, -128) from the subnormal-code dot products.
//   * Each lane keeps a ring of D units x R rows of payload in flight: slot d
//     is refilled with the unit D steps ahead as soon as it is unpacked, and
//     the first D loads go out before the x staging, so the weight stream
//     never waits on the LDS phase. Units are unpacked in registers
//     (v_perm_b32 into fp16 subnormals) and accumulated with v_dot2_f32_f16.
//     A block's dot product is scaled by its fp16 scale once, as the
//     reference does (quantization.py:199, 215).
//   * Partial row sums are reduced across the G lanes with cross-lane
//     shuffles; lane 0 of a group adds the bias and stores fp16 or fp32.
#include "svq_device.h"
#include "svq_launch.h"

namespace svq {

constexpr int kThreads = 256;
constexpr int kWavesPerGroup = kThreads / 64;
// A buffer offset past every per-wave range (the C ABI keeps a wave's rows
// below 2^31 bytes): loads there return zeros and touch no memory.
constexpr uint32_t kOutOfRange = 0x80000000u;

template <int QT, int M, int R, int D>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs a) {
  using T = QTraits<QT>;
  constexpr int P = T::kUnitWeights / 8;   // 16-byte activation pieces per unit
  constexpr int XW = T::kUnitWeights / 2;  // activation dwords per unit
  extern __shared__ u32x4 lds[];

  const int n = a.n, k = a.k;
  const int kb = k >> 5;
  const int units = kb * T::kUnitsPerBlock;
  const int lg_g = a.lg_g;
  const int G = 1 << lg_g;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane & (G - 1);
  const int rg = lane >> lg_g;
  const int rows_per_wave = (64 >> lg_g) * R;
  const int row_wave0 = (blockIdx.x * kWavesPerGroup + wave) * rows_per_wave;
  const bool wave_active = row_wave0 < n;
  const int row_lane0 = row_wave0 + rg * R;
  const uint32_t row_bytes = (uint32_t)kb * T::kBlockQ;

  // Per-wave buffer resources over exactly the wave's rows; lanes address
  // with 32-bit offsets from them. Rows past n are clamped to n - 1 (loaded,
  // never stored).
  const int wave_rows = wave_active ? min(rows_per_wave, n - row_wave0) : 0;
  const __amdgpu_buffer_rsrc_t qr =
      make_rsrc(a.q + (size_t)(wave_active ? row_wave0 : 0) * row_bytes,
                (uint32_t)wave_rows * row_bytes);
  const __amdgpu_buffer_rsrc_t sr =
      make_rsrc(a.s + (size_t)(wave_active ? row_wave0 : 0) * kb,
                (uint32_t)wave_rows * (uint32_t)kb * 2u);
  uint32_t qoff[R], soff[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    int row = row_lane0 + r;
    row = row < n ? row : n - 1;
    const int rel = wave_active ? row - row_wave0 : 0;
    qoff[r] = (uint32_t)rel * row_bytes;
    soff[r] = (uint32_t)rel * (uint32_t)kb * 2u;
  }

  float acc[R][M];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.f;
  // Bias of the lane's rows, fetched now so its latency overlaps the stream.
  float bias[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = min(row_lane0 + r, n - 1);
    bias[r] = a.bias && wave_active ? half_bits_to_float(a.bias[row]) : 0.f;
  }

  const int chunk = a.chunk_units;
  u32x4* xs = lds;
  float* sxs = reinterpret_cast<float*>(lds + M * P * chunk);
  // Ring of D in-flight units per row: slot d holds the payload dwords and
  // scale bits of one unit for each of the R rows. Every slot load is issued
  // unconditionally; a load with nothing to fetch gets an offset past the
  // buffer's range, which returns zeros without a memory access. (A
  // conditional load would make the compiler merge register values at the
  // branch join and wait for the load there.)
  uint32_t w[D][R][T::kWords];
  uint32_t sc[D][R];
  auto load_slot = [&](int d, int cu0, int u, bool valid) {
    const uint32_t ug = (uint32_t)(cu0 + u);
    // Added rather than selected: valid offsets are below 2^31, so this moves
    // an invalid load out of range without giving the compiler a branch.
    const uint32_t oob = (uint32_t)(!valid) * kOutOfRange;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      load_unit_buf<QT>(qr, qoff[r] + ug * T::kUnitBytes + oob, w[d][r]);
      sc[d][r] = __builtin_amdgcn_raw_buffer_load_b16(
          sr, soff[r] + (ug / T::kUnitsPerBlock) * 2u + oob, 0, 0);
    }
  };

  for (int cu0 = 0; cu0 < units; cu0 += chunk) {
    const int cun = min(chunk, units - cu0);
    // Units of this chunk handled by this lane: g, g + G, ...
    const int niter = g < cun ? (cun - g + G - 1) >> lg_g : 0;
    // The first D loads are issued before the x staging and its barriers, so
    // the two memory latencies overlap.
    if (wave_active) {
#pragma unroll
      for (int d = 0; d < D; ++d) load_slot(d, cu0, g + d * G, d < niter);
    }
    if (cu0 > 0) __syncthreads();  // previous chunk fully consumed
    stage_x<QT, M, kThreads>(a.x, k, cu0, cun, chunk, xs, sxs);

    if (wave_active) {
      for (int i = 0; i < niter; i += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
          const int it = i + d;
          const int u = g + it * G;
          if (it < niter) {
            uint32_t pk[R][XW];
#pragma unroll
            for (int r = 0; r < R; ++r) unpack<QT>(w[d][r], pk[r]);
            float dsc[R];
#pragma unroll
            for (int r = 0; r < R; ++r) dsc[r] = half_bits_to_float((uint16_t)sc[d][r]);
#pragma unroll
            for (int m = 0; m < M; ++m) {
              uint32_t xv[XW];
#pragma unroll
              for (int p = 0; p < P; ++p) {
                const u32x4 v = xs[(m * P + p) * chunk + u];
                xv[4 * p] = v.x; xv[4 * p + 1] = v.y;
                xv[4 * p + 2] = v.z; xv[4 * p + 3] = v.w;
              }
              const float off = sxs[m * chunk + u];
#pragma unroll
              for (int r = 0; r < R; ++r)
                acc[r][m] = __builtin_fmaf(unit_dot<QT>(pk[r], xv, off), dsc[r], acc[r][m]);
            }
          }
          // Refill the slot with the unit D steps ahead.
          load_slot(d, cu0, u + D * G, it + D < niter);
        }
      }
    }
  }

  if (!wave_active) return;
  // Reduce each row's partial sums over its G lanes.
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float v = acc[r][m];
      for (int off = G >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
      acc[r][m] = v;
    }
  if (g != 0) return;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row_lane0 + r;
    if (row >= n) break;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float v = __builtin_fmaf(acc[r][m], T::kOutScale, bias[r]);
      store_y(a, m, row, v);
    }
  }
}

// LDS bytes per staged unit and activation row: P 16-byte pieces + one float.
template <int QT>
constexpr int lds_unit_bytes() { return QTraits<QT>::kUnitWeights * 2 + 4; }

template <int QT, int M, int R, int D>
static hipError_t launch_one(const GemvArgs& a, const GemvShape& sh,
                             hipStream_t stream) {
  const size_t lds = (size_t)M * sh.chunk_units * lds_unit_bytes<QT>();
  hipLaunchKernelGGL((gemv_kernel<QT, M, R, D>), dim3(sh.groups),
                     dim3(kThreads), lds, stream, a);
  return hipGetLastError();
}

template <int QT, int M>
static hipError_t launch_m(const GemvArgs& a, const GemvShape& sh,
                           hipStream_t stream) {
  if (sh.rows_per_group == 2) return launch_one<QT, M, 2, 4>(a, sh, stream);
  return launch_one<QT, M, 1, 8>(a, sh, stream);
}

template <int QT>
static hipError_t launch_q(const GemvArgs& a, const GemvShape& sh,
                           hipStream_t stream) {
  switch (sh.m) {
    case 1: return launch_m<QT, 1>(a, sh, stream);
    case 2: return launch_m<QT, 2>(a, sh, stream);
    case 3: return launch_m<QT, 3>(a, sh, stream);
    case 4: return launch_m<QT, 4>(a, sh, stream);
    case 5: return launch_m<QT, 5>(a, sh, stream);
    case 6: return launch_m<QT, 6>(a, sh, stream);
    case 7: return launch_m<QT, 7>(a, sh, stream);
    case 8: return launch_m<QT, 8>(a, sh, stream);
  }
  return hipErrorInvalidValue;
}

int lds_bytes_per_unit(int qtype) {
  switch (qtype) {
    case 4: return lds_unit_bytes<4>();
    case 5: return lds_unit_bytes<5>();
    case 8: return lds_unit_bytes<8>();
  }
  return 0;
}

int units_per_block(int qtype) { return qtype == 8 ? 2 : 1; }

hipError_t launch_gemv(const GemvArgs& a, const GemvShape& sh, int qtype,
                       hipStream_t stream) {
  switch (qtype) {
    case 4: return launch_q<4>(a, sh, stream);
    case 5: return launch_q<5>(a, sh, stream);
    case 8: return launch_q<8>(a, sh, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace svq
