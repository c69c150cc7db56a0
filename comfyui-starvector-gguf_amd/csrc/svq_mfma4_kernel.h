// Kernel template of the streaming fused GGUF SoA dequantize + GEMV on the
// 4x4x4 matrix cores, shared by the translation units that instantiate it
// (svq_gemv_mfma4.hip: M = 1..4, svq_gemv_mfma4_wide.hip: M = 5..8, built in
// parallel). Everything here has internal linkage.
//
// Streaming fused GGUF SoA dequantize + GEMV with the dot products on the
// matrix cores (v_mfma_f32_4x4x4_16b_f16), for 1 <= M <= 8.
//
// Same arithmetic as the reference `_soa_gemv` (quantization.py:171-229): a
// block's integer-code dot product in fp32, multiplied once by the block's
// fp16 scale; bias added in fp32; fp16 or fp32 out.
//
// The 4x4x4 MFMA computes 16 independent 4 x 4 x 4 products per wave: lanes
// 4b..4b+3 form block b, and lane 4b + i supplies row i of the block's A (4
// k values), column i of its B (4 k values) and receives column i of its D
// (4 rows). Here lane (b = lane / 4, i = lane % 4) streams the units b, b+16,
// b+32, ... of weight row i of its row set, exactly like 16 lanes per row of
// the vector streaming kernel, and
//   A row i = x[i % M] over the unit's 4 k positions of the step,
//   B column i = those 4 weights of row i as fp16 subnormal codes,
//   C = offset * sum(x[m] over the unit), so the block's D column i holds the
//       unit's dot product of weight row i with every activation row m < 4.
// Eight chained MFMAs cover a 32-weight unit (four for a Q8_0 half block);
// then acc[m] += D[m] * scale. The per-weight cost on the vector units is the
// unpack alone: the M dot products per weight move to the matrix cores.
// For 5 <= M <= 8 every unpacked B meets two A halves, x rows 0..3 and
// 4..7 (rows >= M repeat a valid row and are ignored), in two independent
// MFMA chains: the unpack is shared by all M rows.
//
// Everything else follows the vector streaming kernel (svq_gemv_stream.hip):
// persistent waves over row tiles, x and the offset sums staged in LDS once per
// workgroup, a ring of D units per row in flight across tiles, out-of-range
// loads for the ragged ends. Units past the end of a row keep every lane in
// the MFMA (it runs for the whole wave): their payload and scale load as
// zeros and their x reads are clamped to the last unit, so they add nothing.
#pragma once

#include "svq_device.h"
#include "svq_launch.h"

namespace svq {

namespace {

typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr uint32_t kOutOfRange = 0x80000000u;  // past every buffer range (< 2^31 bytes)

// Phase stamps (100 MHz real-time clock) of lane 0 of every wave, in builds
// with SVQ_TIMELINE only (libsvq_timeline.so); nothing otherwise.
#if SVQ_TIMELINE
#define SVQ_STAMP(slot, value)                                    \
  do {                                                            \
    if (stamps_ && (threadIdx.x & 63) == 0) stamps_[slot] = (value); \
  } while (0)
#else
#define SVQ_STAMP(slot, value) \
  do {                         \
  } while (0)
#endif
constexpr int kSlots = 16;                     // unit slots per row: MFMA blocks per wave

// Output and offset scaling: Q4_0 and Q5_0 codes are placed as 16 * code.
template <int QT> struct Mfma4Traits;
template <> struct Mfma4Traits<4> {
  static constexpr int kSxMul = 16;
  static constexpr float kOutScale = 0x1p20f;
};
template <> struct Mfma4Traits<5> {
  static constexpr int kSxMul = 1;  // QTraits<5> already counts 16 * code
  static constexpr float kOutScale = 0x1p20f;
};
template <> struct Mfma4Traits<8> {
  static constexpr int kSxMul = 1;
  static constexpr float kOutScale = 0x1p24f;
};

// x pieces per thread loaded before the weight prologue: all of x for K =
// 4608 at M <= 4 with 256 threads, so x arrives in one load round trip (at M
// = 3..4 batches of 4 took three in a row); 10 at M = 8 (two round trips for
// K = 4608 instead of five: 0.3-1.0 us faster on the 8B shapes); 4 at M =
// 5..7, where 10 measured up to 1.5 us slower.
template <int QT, int M>
constexpr int kStage4Batch =
    M <= 4 ? M * 144 * (QTraits<QT>::kUnitWeights / 8) * QTraits<QT>::kUnitsPerBlock / 256 + 1
           : M == 8 ? 10 : 4;

// Sum of v over the 16 lanes b * 4 + i (b = 0..15) of each i: DPP rotations
// by 4 and 8 inside each 16-lane row, then the gfx950 lane swaps across rows.
__device__ __forceinline__ float slot_sum(float v) {
  auto ror = [](float f, auto ctrl) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(
        __builtin_bit_cast(int, f), decltype(ctrl)::value, 0xf, 0xf, false));
  };
  v += ror(v, std::integral_constant<int, 0x124>{});  // row_ror:4
  v += ror(v, std::integral_constant<int, 0x128>{});  // row_ror:8
  int i = __builtin_bit_cast(int, v);
  auto r = __builtin_amdgcn_permlane16_swap(i, i, false, false);
  v = __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
  i = __builtin_bit_cast(int, v);
  r = __builtin_amdgcn_permlane32_swap(i, i, false, false);
  return __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
}

// U: consecutive units per lane per step. U = 3 (Q5_0 only) reads a lane's
// 60 bytes as three 16-byte loads and one 12-byte load and its three scales as
// 2 + 4 bytes: 6 loads per 3 units instead of 9, which the memory pipeline
// serves about 13% faster. It needs units % 48 == 0 (K = 4608, 18432, ...).
// SP (short prologue): one weight ring step before x is staged.
template <int QT, int M, int R, int D, int WPG, int U, bool LN, bool SP = false>
__global__ __launch_bounds__(WPG * 64) void gemv_mfma4_kernel(GemvArgs a) {
  static_assert(M >= 1 && M <= 8, "A has 4 rows: one half for M <= 4, two for M <= 8");
  constexpr int H = M > 4 ? 2 : 1;  // A halves (MFMA chains per unpacked B)
  static_assert(U == 1 || (U == 3 && QT != 8) || (U == 2 && QT == 8),
                "consecutive units per lane: three Q4_0 / Q5_0 blocks or one Q8_0 block");
  using T = QTraits<QT>;
  constexpr int kWordsU = U * T::kWords;  // payload dwords per lane per step
  constexpr int J = T::kUnitWeights / 4;  // MFMAs per unit
  extern __shared__ u32x4 lds[];
  __shared__ u32x2 q5_table[QT == 5 ? 256 : 1];

#if SVQ_TIMELINE
  const unsigned long long t_entry = __builtin_amdgcn_s_memrealtime();
  unsigned long long* stamps_ =
      a.stamps ? a.stamps + ((blockIdx.y * gridDim.x + blockIdx.x) * WPG + (threadIdx.x >> 6)) *
                                kTimelineSlots
               : nullptr;
#endif
  // Every argument the work split and the first loads need, pinned in
  // scalar registers before the first branch: the compiler otherwise loads
  // each one just ahead of its first use, behind the branches, one scalar
  // memory round trip per branch on the way to the first x load.
  int n = a.n, k = a.k, a_units = a.units, a_tiles = a.tiles, a_groups = a.tile_groups;
  int a_wave_major = a.wave_major, a_tiles_hi = a.tiles_hi, a_tiles_full = a.tiles_full;
  int a_steps = a.steps, a_lg_ksplit = a.lg_ksplit;
  int grid_x = (int)gridDim.x, grid_y = (int)gridDim.y;
  const uint16_t* a_x = a.x;
  const uint8_t* a_q = a.q;
  const uint16_t* a_s = a.s;
  const uint16_t* a_bias = a.bias;
  const uint16_t* a_ln_w = LN ? a.ln_w : nullptr;
  const uint16_t* a_ln_b = LN ? a.ln_b : nullptr;
  asm volatile(""
               : "+s"(n), "+s"(k), "+s"(a_units), "+s"(a_tiles), "+s"(a_groups),
                 "+s"(a_wave_major), "+s"(a_tiles_hi), "+s"(a_tiles_full), "+s"(a_steps),
                 "+s"(a_lg_ksplit), "+s"(grid_x), "+s"(grid_y), "+s"(a_x), "+s"(a_q),
                 "+s"(a_s), "+s"(a_bias), "+s"(a_ln_w), "+s"(a_ln_b));
  const int kb = k >> 5;
  // K slices across workgroups (a.partial set, gridDim.x = a.slices >= 2):
  // workgroup (slice, b) takes that slice of every row -- units ubase ..
  // ubase + units, x staged for that slice only -- and writes raw partial
  // sums. Otherwise one slice: the whole row. The slices of a row set are
  // consecutive in dispatch order.
  const int SL = grid_x;
  const int slice = (int)blockIdx.x;
  const int units = a_units;
  const int ubase = slice * units;
  const int bx = (int)blockIdx.y;  // workgroup within its slice
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int slot = lane >> 2;  // MFMA block: the unit slot of this lane
  const int ri = lane & 3;     // row of the row set; also the A row it supplies
  int m_a[H];                  // activation row it supplies per half (rows >= M repeat)
#pragma unroll
  for (int h = 0; h < H; ++h) m_a[h] = (4 * h + ri) % M;
  // Work split: the WPG waves of a workgroup are P tile slots x S K-ranges;
  // wave (p, sk) streams steps [st0, st1) of each tile of slot p. With S > 1
  // workgroup g processes tile groups g, g + G, ... (P tiles each) and the S
  // partial sums of a tile meet in LDS at the end of its group.
  const int lg_s = a_lg_ksplit, S = 1 << lg_s, P = WPG >> lg_s;
  const int p_id = wave >> lg_s, sk = wave & (S - 1);
  const int tile_rows = 4 * R;
  const int tiles = a_tiles;
  const int groups = a_groups;
  const int G = grid_y;
  // At most one tile per wave (S = 1): wave-major tiles (wave p of
  // workgroup g owns tile wv = p * G + g), which spreads the idle waves of a
  // short matrix over all workgroups, hence over all CUs. Otherwise workgroup
  // g walks tile groups g, g + G, ... (P consecutive tiles each), which keeps
  // the rows a workgroup streams at a time together; with S > 1 the S waves
  // of a tile slot meet at a barrier per tile, so every wave of a workgroup
  // walks the same number of tile groups.
  const int WV = P * G;
  const bool wave_major = a_wave_major != 0;
  const int wv = p_id * G + bx;
  // Tile groups bx, bx + G, ... below `groups`: tiles_hi of them for
  // workgroups below tiles_full, one fewer from there (none past groups).
  const int my_tiles = wave_major ? (wv < tiles ? 1 : 0)
                                  : (bx < a_tiles_full ? a_tiles_hi : a_tiles_hi - 1);
  const int niter_all = a_steps;
  const int st0 = (sk * niter_all) >> lg_s, st1 = ((sk + 1) * niter_all) >> lg_s;
  const int steps = my_tiles * (st1 - st0);
  auto tile_of = [&](int j) { return wave_major ? wv + j * WV : (bx + j * G) * P + p_id; };
  // A workgroup without tiles leaves before staging x (the same decision for
  // all its waves): wave-major, when its first wave (wv = g) has none;
  // otherwise when it has no tile group.
#if SVQ_TIMELINE
  SVQ_STAMP(0, t_entry);
  SVQ_STAMP(5, 0ull);
  SVQ_STAMP(7, __builtin_amdgcn_s_memrealtime());
#endif
  if (bx >= (wave_major ? tiles : groups)) return;
  const uint32_t row_bytes = (uint32_t)kb * T::kBlockQ;

  const __amdgpu_buffer_rsrc_t qr = make_rsrc(a_q, (uint32_t)n * row_bytes);
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(a_s, (uint32_t)n * (uint32_t)kb * 2u);
  const __amdgpu_buffer_rsrc_t br = make_rsrc(a_bias, a_bias ? (uint32_t)n * 2u : 0u);

  constexpr int XP = T::kUnitWeights / 8;  // 16-byte x pieces per unit
  // LDS: x pieces, LayerNorm parameters (if any), offset sums, split-K sums.
  const bool ln = LN && (a_ln_w || a_ln_b);
  u32x4* xs = lds;
  u32x4* lns = xs + M * XP * units;
  float* sxs = reinterpret_cast<float*>(lns + (ln ? 2 * ((k / 8 + 63) / 64 * 64) : 0));
  float* part = sxs + M * units;  // [2][WPG][R][M][4] split-K partial sums

  // Row offsets of this lane's R rows in tile `tile` (rows past n: out of
  // range, so they load zeros).
  auto row_offsets = [&](int tile, uint32_t (&qo)[R], uint32_t (&so)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = tile * tile_rows + r * 4 + ri;
      const bool ok = tile < tiles && row < n;
      const uint32_t rr = ok ? (uint32_t)row : 0u;
      const uint32_t oob = (uint32_t)(!ok) * kOutOfRange;
      qo[r] = rr * row_bytes + oob;
      so[r] = rr * (uint32_t)kb * 2u + oob;
    }
  };

  uint32_t w[D][R][kWordsU];
  uint32_t sc[D][R][U == 3 ? 2 : 1];  // U = 3: the 8 bytes that hold blocks u .. u + 2's scales
  int pj = 0, pit = st0;
  uint32_t pqo[R], pso[R];
  row_offsets(tile_of(0), pqo, pso);
  auto issue = [&](int d) {
    const int u = U * (slot + pit * kSlots);
    const bool valid = pj < my_tiles && u < units;
    const uint32_t oob = (uint32_t)(!valid) * kOutOfRange;
    const uint32_t ug = (uint32_t)(ubase + u);  // unit within the whole row
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if constexpr (U == 3 && QT == 5) {
        // Three 20-byte blocks: 60 contiguous bytes as 3 x 16 + 12.
        typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
        const uint32_t off = pqo[r] + ug * 20u + oob;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
          const u32x4 v = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, off + 16u * c, 0, 0));
          w[d][r][4 * c] = v.x; w[d][r][4 * c + 1] = v.y;
          w[d][r][4 * c + 2] = v.z; w[d][r][4 * c + 3] = v.w;
        }
        const u32x3 t = __builtin_bit_cast(
            u32x3, __builtin_amdgcn_raw_buffer_load_b96(qr, off + 48u, 0, 0));
        w[d][r][12] = t.x; w[d][r][13] = t.y; w[d][r][14] = t.z;
      } else if constexpr (U > 1) {
        // U consecutive 16-byte units: U x 16 contiguous bytes.
        const uint32_t off = pqo[r] + ug * 16u + oob;
#pragma unroll
        for (int c = 0; c < U; ++c) {
          const u32x4 v = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, off + 16u * c, 0, 0));
          w[d][r][4 * c] = v.x; w[d][r][4 * c + 1] = v.y;
          w[d][r][4 * c + 2] = v.z; w[d][r][4 * c + 3] = v.w;
        }
      }
      if constexpr (U == 3) {
        // Three consecutive blocks (one unit each): their three scales, the 6
        // bytes at byte 0 or 2 of the 8 dword-aligned bytes that hold them
        // (rows start dword-aligned: kb is even), in one load.
        const uint32_t soff = (pso[r] + ug * 2u + oob) & ~3u;
        const u32x2 sv =
            __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(sr, soff, 0, 0));
        sc[d][r][0] = sv.x;
        sc[d][r][1] = sv.y;
      } else if constexpr (U == 2) {
        // The two halves of one Q8_0 block (u even): one scale.
        sc[d][r][0] = __builtin_amdgcn_raw_buffer_load_b16(
            sr, pso[r] + (ug / 2u) * 2u + oob, 0, 0);
      } else {
        // 16 lanes of a row read 16 consecutive units: whole cache lines.
        load_unit_buf<QT, QT == 5 ? 0 : kLoadNonTemporal>(qr, pqo[r] + ug * T::kUnitBytes + oob,
                                                          w[d][r]);
        sc[d][r][0] = __builtin_amdgcn_raw_buffer_load_b16(
            sr, pso[r] + (ug / T::kUnitsPerBlock) * 2u + oob, 0, 0);
      }
    }
    if (++pit == st1) {
      pit = st0;
      ++pj;
      row_offsets(tile_of(pj), pqo, pso);
    }
  };

  auto load_bias = [&](int tile, uint32_t (&bb)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = tile * tile_rows + r * 4 + ri;
      const uint32_t oob = (uint32_t)(!(tile < tiles && row < n)) * kOutOfRange;
      bb[r] = __builtin_amdgcn_raw_buffer_load_b16(br, (uint32_t)(row < n ? row : 0) * 2u + oob,
                                                   0, 0);
    }
  };

  // x and bias loads first, then the weight prologue, then x is written to
  // LDS (vector loads retire in issue order).
  XStager<QT, M, WPG * 64, kStage4Batch<QT, M>, Mfma4Traits<QT>::kSxMul, LN> st(a_x, k, ubase, units,
                                                                               units);
  st.set_layer_norm(a_ln_w, a_ln_b, a.ln_eps);
#if SVQ_TIMELINE
  st.stamps = stamps_;
#endif
  // The x and bias loads, and later the staging's finish (LDS writes,
  // LayerNorm, barrier), run at raised wave priority, so they win the SIMD's
  // issue arbitration over the other workgroup's weight stream. Measured in
  // one process against no raise: Q5_0 M = 2 c_fc 18432 x 4608 15.3 -> 14.7
  // us, lm_head 31.3 -> 30.5 us, the five-matrix step 77.0 -> 76.1 us; 8B
  // beam-2 decode 508 -> 518 steps/s, 1B 990 -> 1000 (the loads alone: 514
  // and 996; priority 1 and 3 alike). Raised from the x loads through the
  // finish, weight prologue included: step 75.4 us, but 8B decode 510 and 1B
  // 975 steps/s (both decoders are Q4_0), so only Q5_0 keeps the raise over
  // its weight prologue (against dropping it there: qkv 5632 x 4608 7.74 ->
  // 7.47 us, o_proj 7.31 -> 7.12 us, step 76.2 -> 75.7 us; Q4_0 and Q8_0
  // shapes and both decoders unchanged).
  constexpr bool kRaisedPrologue = QT == 5;
  __builtin_amdgcn_s_setprio(1);
  st.begin(lns);
  SVQ_STAMP(6, __builtin_amdgcn_s_memrealtime());
  uint32_t bias_bits[R];  // before the prologue: waiting for it waits for x only
  load_bias(tile_of(0), bias_bits);
  // The fifth-bit table is built while x is in flight; the staging's
  // barrier orders its LDS writes before the first lookup.
  if constexpr (QT == 5) build_q5_table(q5_table, threadIdx.x, WPG * 64);
  if constexpr (!kRaisedPrologue) __builtin_amdgcn_s_setprio(0);
  // Weight ring steps issued before x is staged; the rest follow the staging.
  // The x loads of the CU's other workgroup queue behind every weight load
  // issued here. Q4_0 three-block lanes issue one step first (measured in one
  // process at M = 2: qkv 5632 x 4608 7.7 -> 7.3 us, c_fc 18432 x 4608 13.5
  // -> 12.8 us; 8B beam-2 decode 486 -> 494 steps/s), and so do Q5_0 ones
  // with SP, which the host sets when every tile slot has at most one row
  // tile (qkv 8.8 -> 8.1 us, o_proj 8.3 -> 7.8 us; with more tiles per slot
  // one step first lost: c_fc 15.6 -> 15.8, c_proj's slices 18.8 -> 19.1,
  // lm_head 31.5 -> 32.6 us). One-unit lanes and Q8_0 whole-block lanes
  // issue half their ring first (one step first lost on short matrices:
  // 2304 x 2048 at M = 2, Q4_0 4.9 -> 5.7 us, Q8_0 4.6 -> 5.1 us; half the
  // ring gains up to 0.6 us at K = 2048 and 8192, e.g. Q4_0 49152 x 2048 at
  // M = 2 14.5 -> 13.9 us, Q5_0 2048 x 8192 8.2 -> 7.7 us, and loses at most
  // 0.4 us). Q5_0 three-block lanes without SP keep the whole ring first.
  // The count is a compile-time constant: with a run-time count the
  // compiler's wait counts turn conservative and every variant lost up to
  // 1 us.
  constexpr int kPre = (SP || (QT == 4 && U == 3)) ? 1 : U == 3 ? D : D / 2;
#pragma unroll
  for (int d = 0; d < kPre; ++d) issue(d);
  if constexpr (!kRaisedPrologue) __builtin_amdgcn_s_setprio(1);
  st.finish(xs, sxs, lns);
  __builtin_amdgcn_s_setprio(0);
#pragma unroll
  for (int d = kPre; d < D; ++d) issue(d);
  SVQ_STAMP(1, __builtin_amdgcn_s_memrealtime());
  SVQ_STAMP(5, (unsigned long long)my_tiles);

  float acc[R][M];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.f;

  int cj = 0, cit = st0;
  for (int s = 0; s < steps; s += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      if (s + d < steps) {
#pragma unroll
        for (int q = 0; q < U; ++q) {
          const int u = min(U * (slot + cit * kSlots) + q, units - 1);
          // A: 4 k values of activation row m_a[h] per MFMA (shared by the R rows).
          uint32_t xa[H][XP * 4];
#pragma unroll
          for (int h = 0; h < H; ++h)
#pragma unroll
            for (int p = 0; p < XP; ++p) {
              const u32x4 v = xs[(m_a[h] * XP + p) * units + u];
              xa[h][4 * p] = v.x; xa[h][4 * p + 1] = v.y;
              xa[h][4 * p + 2] = v.z; xa[h][4 * p + 3] = v.w;
            }
          // C: the offset term of every activation row (rows >= M: zero).
          f4_t cv[H];
#pragma unroll
          for (int h = 0; h < H; ++h)
#pragma unroll
            for (int m = 0; m < 4; ++m) cv[h][m] = 4 * h + m < M ? sxs[(4 * h + m) * units + u] : 0.f;
#pragma unroll
          for (int r = 0; r < R; ++r) {
            uint32_t uw[T::kWords];
#pragma unroll
            for (int i = 0; i < T::kWords; ++i) uw[i] = w[d][r][q * T::kWords + i];
            uint32_t pk[T::kUnitWeights / 2];
            if constexpr (QT == 4) unpack_q4_x16(uw, pk);
            else if constexpr (QT == 5) unpack_q5_table(uw, pk, q5_table);
            else unpack<QT>(uw, pk);
            f4_t dv[H];
#pragma unroll
            for (int h = 0; h < H; ++h) dv[h] = cv[h];
#pragma unroll
            for (int j = 0; j < J; ++j) {
              u32x2 bv;
              bv.x = pk[2 * j]; bv.y = pk[2 * j + 1];
#pragma unroll
              for (int h = 0; h < H; ++h) {
                u32x2 av;
                av.x = xa[h][2 * j]; av.y = xa[h][2 * j + 1];
                dv[h] = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(h4_t, av),
                                                           __builtin_bit_cast(h4_t, bv), dv[h], 0, 0,
                                                           0);
              }
            }
            // Scale of unit q: half q of the 8 loaded bytes, after the 2-byte
            // lead-in when the first unit's index is odd.
            const uint32_t sbits =
                U != 3 ? sc[d][r][0]
                       : (uint32_t)((((uint64_t)sc[d][r][1] << 32) | sc[d][r][0]) >>
                                    (16 * q + 16 * ((ubase + U * (slot + cit * kSlots)) & 1)));
            const float scale = half_bits_to_float((uint16_t)sbits);
#pragma unroll
            for (int m = 0; m < M; ++m)
              acc[r][m] = __builtin_fmaf(dv[m / 4][m % 4], scale, acc[r][m]);
          }
        }
      }
      issue(d);  // refill with the step D ahead (out of range past the end)
      if (s == 0 && d == 0) SVQ_STAMP(2, __builtin_amdgcn_s_memrealtime());
      if (s + d < steps && ++cit == st1) {
        // Tile done: add the 16 unit slots of each row (and the S K-ranges),
        // store, next tile.
        const int tile = tile_of(cj);
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int m = 0; m < M; ++m) acc[r][m] = slot_sum(acc[r][m]);
        if (cj == 0) SVQ_STAMP(3, __builtin_amdgcn_s_memrealtime());
        if (S > 1) {
          float* buf = part + (cj & 1) * WPG * R * M * 4;
          if (slot == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
              for (int m = 0; m < M; ++m) buf[((wave * R + r) * M + m) * 4 + ri] = acc[r][m];
          }
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
          __builtin_amdgcn_s_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
          if (sk == 0 && slot == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
              for (int m = 0; m < M; ++m) {
                float v = 0.f;
                for (int o = 0; o < S; ++o) v += buf[(((p_id * S + o) * R + r) * M + m) * 4 + ri];
                acc[r][m] = v;
              }
          }
        }
        if (slot == 0 && sk == 0) {
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const int row = tile * tile_rows + r * 4 + ri;
            if (row < n) {
              if (SL > 1) {  // raw slice sums; split_finish scales, biases and stores
#pragma unroll
                for (int m = 0; m < M; ++m)
                  a.partial[((size_t)slice * M + m) * n + row] = acc[r][m];
              } else {
                const float b = half_bits_to_float((uint16_t)bias_bits[r]);
#pragma unroll
                for (int m = 0; m < M; ++m) {
                  const float v = __builtin_fmaf(acc[r][m], Mfma4Traits<QT>::kOutScale, b);
                  store_y(a, m, row, v);
                }
              }
            }
          }
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int m = 0; m < M; ++m) acc[r][m] = 0.f;
        cit = st0;
        ++cj;
        load_bias(tile_of(cj), bias_bits);
      }
    }
  }
  SVQ_STAMP(4, __builtin_amdgcn_s_memrealtime());
}

template <int QT, int M, int R, int D, int U, bool LN, bool SP>
const void* mfma4_kernel_ptr() {
  return reinterpret_cast<const void*>(
      &gemv_mfma4_kernel<QT, M, R, D, kStreamWavesPerGroup, U, LN, SP>);
}

template <int QT, int M, int R, int D, int U, bool LN, bool SP>
hipError_t mfma4_launch(const GemvArgs& a, int groups, size_t lds, hipStream_t stream) {
  // groups = K slices (gridDim.x) x workgroups per slice (gridDim.y).
  const int sl = a.partial ? a.slices : 1;
  hipLaunchKernelGGL((gemv_mfma4_kernel<QT, M, R, D, kStreamWavesPerGroup, U, LN, SP>),
                     dim3(sl, groups / sl), dim3(kStreamWavesPerGroup * 64), lds, stream, a);
  return hipGetLastError();
}

// One (R, D, U) variant, with or without the LayerNorm staging.
template <int QT, int M, int R, int D, int U, bool SP = false>
hipError_t mfma4_variant(const GemvArgs& a, bool ln, int groups, size_t lds, hipStream_t stream,
                         const void** fn) {
  if (fn) {
    *fn = ln ? mfma4_kernel_ptr<QT, M, R, D, U, true, SP>()
             : mfma4_kernel_ptr<QT, M, R, D, U, false, SP>();
    return hipSuccess;
  }
  return ln ? mfma4_launch<QT, M, R, D, U, true, SP>(a, groups, lds, stream)
            : mfma4_launch<QT, M, R, D, U, false, SP>(a, groups, lds, stream);
}

// rows 1: one row set per lane with an 8-deep ring; rows 2: two row sets
// (sharing each x read) with a 4-deep ring; rows 3: one row set, consecutive
// units per lane: three Q4_0 / Q5_0 blocks with a 3-deep ring (9 units in
// flight) or one Q8_0 block (two units) with a 4-deep ring.
template <int QT, int M>
hipError_t mfma4_dispatch_r(const GemvArgs& a, bool ln, int rows, int groups, size_t lds,
                            hipStream_t stream, const void** fn) {
  if (rows == 3) {
    if constexpr (QT == 8) return mfma4_variant<QT, M, 1, 4, 2>(a, ln, groups, lds, stream, fn);
    else if constexpr (QT == 5)
      return a.short_prologue ? mfma4_variant<QT, M, 1, 3, 3, true>(a, ln, groups, lds, stream, fn)
                              : mfma4_variant<QT, M, 1, 3, 3>(a, ln, groups, lds, stream, fn);
    else return mfma4_variant<QT, M, 1, 3, 3>(a, ln, groups, lds, stream, fn);
  }
  if (rows == 2) return mfma4_variant<QT, M, 2, 4, 1>(a, ln, groups, lds, stream, fn);
  return mfma4_variant<QT, M, 1, 8, 1>(a, ln, groups, lds, stream, fn);
}

}  // namespace

// M = 5..8 (two A halves), instantiated in svq_gemv_mfma4_wide.hip.
hipError_t mfma4_dispatch_wide(const GemvArgs& a, bool ln, int qtype, int m, int rows, int groups,
                               size_t lds, hipStream_t stream, const void** fn);

}  // namespace svq
