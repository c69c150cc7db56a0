// Streaming (persistent) fused GGUF SoA dequantize + GEMV for gfx950, the
// main path of svq_gemv whenever the activations x[M, K] fit in LDS.
//
// Same arithmetic as the reference `_soa_gemv` (quantization.py:171-229):
// per 32-weight block, the integer-code dot product is accumulated in fp32 and
// scaled by the block's fp16 scale once; bias added in fp32; fp16 or fp32 out.
//
// Work mapping:
//   * The grid holds at most as many waves as the GPU keeps resident (W, from
//     the occupancy of this kernel, and at most two workgroups per CU). Each
//     workgroup of 4 waves stages x and the per-unit offset sums into LDS
//     once, before its first weight load, and then every wave streams its own
//     rows to the end of the matrix. Wave w of workgroup b is wave
//     wid = b * 4 + w of the grid (wid = w * B + b with B workgroups when
//     there is at most one tile per wave) and owns row tiles
//     t = wid, wid + W, wid + 2W, ...; a tile is (64 / G) * R rows: G lanes
//     share a row and stride over its units, R rows per lane group reuse each
//     activation read from LDS.
//   * A wave's work is one flat sequence of steps (tile, unit-iteration). A
//     ring of D register slots keeps the payload of the next D steps in
//     flight; a slot is refilled as soon as it is unpacked, including across
//     tile boundaries, so the HBM stream never drains between tiles. Loads
//     with nothing to fetch use an offset past the buffer range (zeros, no
//     memory access) instead of a branch.
//   * At the end of each tile the lane group reduces its partial sums with
//     cross-lane shuffles and lane 0 stores R x M outputs; the bias of the
//     next tile is fetched then, a whole tile ahead of its use.
#include "svq_device.h"
#include "svq_launch.h"

namespace svq {

namespace {

constexpr uint32_t kOutOfRange = 0x80000000u;  // past every buffer range (< 2^31 bytes)

// x pieces (16 bytes) per thread loaded before the weight prologue: at
// M <= 2, all of x for K = 4608 with 256 threads; at larger M the batch of 4
// that keeps the register peak of the staging below that of the main loop.
template <int QT, int M>
constexpr int kStageBatch =
    M <= 2 ? M * 144 * (QTraits<QT>::kUnitWeights / 8) * QTraits<QT>::kUnitsPerBlock / 256 + 1
           : 4;

template <int QT, int M, int R, int D, int WPG, bool LN>
__global__ __launch_bounds__(WPG * 64) void gemv_stream_kernel(GemvArgs a) {
  using T = QTraits<QT>;
  constexpr int P = T::kUnitWeights / 8;   // 16-byte activation pieces per unit
  constexpr int XW = T::kUnitWeights / 2;  // activation dwords per unit
  extern __shared__ u32x4 lds[];

  // Every argument the work split and the first loads need, pinned in
  // scalar registers before the first branch (one scalar memory round trip
  // at entry instead of one per branch on the way to the first x load).
  int n = a.n, k = a.k, lg_g = a.lg_g, W = a.waves, grid_x = (int)gridDim.x;
  const uint16_t* a_x = a.x;
  const uint8_t* a_q = a.q;
  const uint16_t* a_s = a.s;
  const uint16_t* a_bias = a.bias;
  const uint16_t* a_ln_w = LN ? a.ln_w : nullptr;
  const uint16_t* a_ln_b = LN ? a.ln_b : nullptr;
  asm volatile(""
               : "+s"(n), "+s"(k), "+s"(lg_g), "+s"(W), "+s"(grid_x), "+s"(a_x), "+s"(a_q),
                 "+s"(a_s), "+s"(a_bias), "+s"(a_ln_w), "+s"(a_ln_b));
  const int kb = k >> 5;
  const int units = kb * T::kUnitsPerBlock;
  const int G = 1 << lg_g;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane & (G - 1);
  const int rg = lane >> lg_g;
  const int tile_rows = (64 >> lg_g) * R;
  const int tiles = (n + tile_rows - 1) / tile_rows;
  // At most one tile per wave: wave-major numbering (wave w of workgroup b
  // is wid = w * gridDim.x + b), which spreads the idle waves of a short
  // matrix over all workgroups, hence over all CUs. Otherwise wid =
  // b * WPG + w: the waves of a workgroup stream neighbouring tiles.
  const bool wave_major = tiles <= W;
  const int wid = wave_major ? wave * grid_x + (int)blockIdx.x
                             : (int)blockIdx.x * WPG + wave;
  const int my_tiles = wid < W ? (tiles - wid + W - 1) / W : 0;
  const int niter = (units + G - 1) >> lg_g;  // unit iterations per tile
  const int steps = my_tiles * niter;
  // A workgroup without tiles leaves before staging x (the same decision for
  // all its waves): its lowest wave number is b (wave-major) or b * WPG.
  if ((wave_major ? (int)blockIdx.x : (int)blockIdx.x * WPG) >= min(W, tiles)) return;
  const uint32_t row_bytes = (uint32_t)kb * T::kBlockQ;

  // Buffer resources over the whole arrays (the C ABI keeps them < 2^31
  // bytes); a missing bias is a zero-length range, so its loads read zeros.
  const __amdgpu_buffer_rsrc_t qr = make_rsrc(a_q, (uint32_t)n * row_bytes);
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(a_s, (uint32_t)n * (uint32_t)kb * 2u);
  const __amdgpu_buffer_rsrc_t br = make_rsrc(a_bias, a_bias ? (uint32_t)n * 2u : 0u);

  // Static LDS: the Q5_0 mask table (a compile-time address, so lookups
  // need no base register). Dynamic LDS: x pieces, then offset sums.
  __shared__ u32x2 q5_table[QT == 5 ? 256 : 1];
  // LDS: x pieces, LayerNorm parameters (if any), offset sums.
  const bool ln = LN && (a_ln_w || a_ln_b);
  u32x4* xs = lds;
  u32x4* lns = xs + M * P * units;
  float* sxs = reinterpret_cast<float*>(lns + (ln ? 2 * ((k / 8 + 63) / 64 * 64) : 0));

  // Row byte offsets of this lane's R rows in tile `tile` (clamped to n - 1:
  // loaded, never stored).
  auto row_offsets = [&](int tile, uint32_t (&qo)[R], uint32_t (&so)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(tile * tile_rows + rg * R + r, n - 1);
      qo[r] = (uint32_t)row * row_bytes;
      so[r] = (uint32_t)row * (uint32_t)kb * 2u;
    }
  };

  // The ring and its prefetch cursor (tile ordinal pj, unit iteration pit).
  uint32_t w[D][R][T::kWords];
  uint32_t sc[D][R];
  int pj = 0, pit = 0;
  uint32_t pqo[R], pso[R];
  row_offsets(wid, pqo, pso);
  auto issue = [&](int d) {
    const int u = g + pit * G;
    const bool valid = pj < my_tiles && u < units;
    // Added rather than selected: a valid offset is below 2^31.
    const uint32_t oob = (uint32_t)(!valid) * kOutOfRange;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      // Lanes of a row read consecutive units: whole cache lines per load.
      load_unit_buf<QT, QT == 5 ? 0 : kLoadNonTemporal>(
          qr, pqo[r] + (uint32_t)u * T::kUnitBytes + oob, w[d][r]);
      sc[d][r] = __builtin_amdgcn_raw_buffer_load_b16(
          sr, pso[r] + (uint32_t)(u / T::kUnitsPerBlock) * 2u + oob, 0, 0);
    }
    if (++pit == niter) {
      pit = 0;
      ++pj;
      row_offsets(wid + pj * W, pqo, pso);
    }
  };

  auto load_bias = [&](int tile, uint32_t (&bb)[R]) {
    const uint32_t oob = (uint32_t)(tile >= tiles) * kOutOfRange;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(tile * tile_rows + rg * R + r, n - 1);
      bb[r] = __builtin_amdgcn_raw_buffer_load_b16(br, (uint32_t)row * 2u + oob, 0, 0);
    }
  };

  // The x loads go out first, then the weight prologue, and only then are the
  // x registers written to LDS. Vector loads retire in issue order, so waiting
  // for x does not wait for the weights, while the weight stream starts one
  // cache round trip earlier than if x were staged completely first. (x loads
  // issued behind the prologue would wait for the whole chip-wide prologue
  // burst.) Pieces beyond the first batch are staged before the ring steps
  // that follow the staging.
  XStager<QT, M, WPG * 64, kStageBatch<QT, M>, 1, LN> st(a_x, k, 0, units, units);
  st.set_layer_norm(a_ln_w, a_ln_b, a.ln_eps);
  st.begin(lns);
  // An 8-deep ring issues half its steps before x is staged and the rest
  // after: the x loads of the CU's other workgroup then queue behind fewer
  // weight loads (M = 1, measured in one process: 49152 x 2048 13.7 -> 12.9
  // us, c_fc 18432 x 4608 12.6 -> 12.4 us; lm_head 49152 x 4608 unchanged).
  // A 4-deep ring issues all four first.
  constexpr int kPre = D > 4 ? 4 : D;
#pragma unroll
  for (int d = 0; d < kPre; ++d) issue(d);
  uint32_t bias_bits[R];
  load_bias(wid, bias_bits);
  // The fifth-bit table is built while x is in flight; the staging's
  // barrier orders its LDS writes before the first lookup.
  if constexpr (QT == 5) build_q5_table(q5_table, threadIdx.x, WPG * 64);
  st.finish(xs, sxs, lns);
#pragma unroll
  for (int d = kPre; d < D; ++d) issue(d);

  float acc[R][M];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.f;

  int cj = 0, cit = 0;  // tile ordinal and unit iteration of the current step
  for (int s = 0; s < steps; s += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      if (s + d < steps) {
        const int u = g + cit * G;
        if (u < units) {
          uint32_t pk[R][XW];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            if constexpr (QT == 5) unpack_q5_table(w[d][r], pk[r], q5_table);
            else unpack<QT>(w[d][r], pk[r]);
          }
          float dsc[R];
#pragma unroll
          for (int r = 0; r < R; ++r) dsc[r] = half_bits_to_float((uint16_t)sc[d][r]);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            uint32_t xv[XW];
#pragma unroll
            for (int p = 0; p < P; ++p) {
              const u32x4 v = xs[(m * P + p) * units + u];
              xv[4 * p] = v.x; xv[4 * p + 1] = v.y;
              xv[4 * p + 2] = v.z; xv[4 * p + 3] = v.w;
            }
            const float off = sxs[m * units + u];
#pragma unroll
            for (int r = 0; r < R; ++r)
              acc[r][m] = __builtin_fmaf(unit_dot<QT>(pk[r], xv, off), dsc[r], acc[r][m]);
          }
        }
      }
      issue(d);  // refill with the step D ahead (out of range past the end)
      if (s + d < steps && ++cit == niter) {
        // Tile done: reduce over the lane group, store, start the next tile.
        const int tile = wid + cj * W;
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int m = 0; m < M; ++m) acc[r][m] = group_sum(acc[r][m], lg_g);
        if (g == 0) {
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const int row = tile * tile_rows + rg * R + r;
            if (row < n) {
              const float b = half_bits_to_float((uint16_t)bias_bits[r]);
#pragma unroll
              for (int m = 0; m < M; ++m) {
                const float v = __builtin_fmaf(acc[r][m], T::kOutScale, b);
                store_y(a, m, row, v);
              }
            }
          }
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int m = 0; m < M; ++m) acc[r][m] = 0.f;
        cit = 0;
        ++cj;
        load_bias(wid + cj * W, bias_bits);
      }
    }
  }
}

template <int QT, int M, int R, int D, int WPG, bool LN>
const void* stream_kernel_ptr() {
  return reinterpret_cast<const void*>(&gemv_stream_kernel<QT, M, R, D, WPG, LN>);
}

template <int QT, int M, int R, int D, int WPG, bool LN>
hipError_t stream_launch(const GemvArgs& a, int groups, size_t lds, hipStream_t stream) {
  hipLaunchKernelGGL((gemv_stream_kernel<QT, M, R, D, WPG, LN>), dim3(groups),
                     dim3(WPG * 64), lds, stream, a);
  return hipGetLastError();
}

// One (R, D) variant, with or without the LayerNorm staging.
template <int QT, int M, int R, int D, int WPG>
hipError_t stream_variant(const GemvArgs& a, bool ln, int groups, size_t lds,
                          hipStream_t stream, const void** fn) {
  if (fn) {
    *fn = ln ? stream_kernel_ptr<QT, M, R, D, WPG, true>()
             : stream_kernel_ptr<QT, M, R, D, WPG, false>();
    return hipSuccess;
  }
  return ln ? stream_launch<QT, M, R, D, WPG, true>(a, groups, lds, stream)
            : stream_launch<QT, M, R, D, WPG, false>(a, groups, lds, stream);
}

// (R, D) pairs: one row per lane group with an 8-deep ring, or two rows with
// a 4-deep ring (8 units in flight per lane either way).
template <int QT, int M, int WPG>
hipError_t stream_dispatch_r(const GemvArgs& a, bool ln, int rows, int groups, size_t lds,
                             hipStream_t stream, const void** fn) {
  if (rows == 2) return stream_variant<QT, M, 2, 4, WPG>(a, ln, groups, lds, stream, fn);
  return stream_variant<QT, M, 1, 8, WPG>(a, ln, groups, lds, stream, fn);
}

template <int QT, int M>
hipError_t stream_dispatch_w(const GemvArgs& a, bool ln, int rows, int wpg, int groups,
                             size_t lds, hipStream_t stream, const void** fn) {
  if (wpg != kStreamWavesPerGroup) return hipErrorInvalidValue;
  return stream_dispatch_r<QT, M, kStreamWavesPerGroup>(a, ln, rows, groups, lds, stream, fn);
}

template <int QT>
hipError_t stream_dispatch_m(const GemvArgs& a, bool ln, int m, int rows, int wpg, int groups,
                             size_t lds, hipStream_t stream, const void** fn) {
  switch (m) {
    case 1: return stream_dispatch_w<QT, 1>(a, ln, rows, wpg, groups, lds, stream, fn);
    case 2: return stream_dispatch_w<QT, 2>(a, ln, rows, wpg, groups, lds, stream, fn);
    case 3: return stream_dispatch_w<QT, 3>(a, ln, rows, wpg, groups, lds, stream, fn);
    case 4: return stream_dispatch_w<QT, 4>(a, ln, rows, wpg, groups, lds, stream, fn);
    case 5: return stream_dispatch_w<QT, 5>(a, ln, rows, wpg, groups, lds, stream, fn);
    case 6: return stream_dispatch_w<QT, 6>(a, ln, rows, wpg, groups, lds, stream, fn);
    case 7: return stream_dispatch_w<QT, 7>(a, ln, rows, wpg, groups, lds, stream, fn);
    case 8: return stream_dispatch_w<QT, 8>(a, ln, rows, wpg, groups, lds, stream, fn);
  }
  return hipErrorInvalidValue;
}

hipError_t stream_dispatch(const GemvArgs& a, bool ln, int qtype, int m, int rows, int wpg,
                           int groups, size_t lds, hipStream_t stream, const void** fn) {
  switch (qtype) {
    case 4: return stream_dispatch_m<4>(a, ln, m, rows, wpg, groups, lds, stream, fn);
    case 5: return stream_dispatch_m<5>(a, ln, m, rows, wpg, groups, lds, stream, fn);
    case 8: return stream_dispatch_m<8>(a, ln, m, rows, wpg, groups, lds, stream, fn);
  }
  return hipErrorInvalidValue;
}

}  // namespace

size_t stream_lds_bytes(int qtype, int m, int k) {
  const int units = (k / 32) * units_per_block(qtype);
  return (size_t)m * units * lds_bytes_per_unit(qtype);
}

const void* stream_kernel(int qtype, int m, int rows, int wpg, bool ln) {
  const void* fn = nullptr;
  GemvArgs unused{};
  (void)stream_dispatch(unused, ln, qtype, m, rows, wpg, 0, 0, nullptr, &fn);
  return fn;
}

hipError_t launch_gemv_stream(const GemvArgs& a, int qtype, int m, int rows, int wpg,
                              int groups, hipStream_t stream) {
  return stream_dispatch(a, a.ln_w || a.ln_b, qtype, m, rows, wpg, groups,
                         stream_lds_bytes(qtype, m, a.k) +
                             layer_norm_lds_bytes(a.k, a.ln_w || a.ln_b),
                         stream, nullptr);
}

}  // namespace svq
