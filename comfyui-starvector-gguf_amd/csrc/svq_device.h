// Device-side building blocks shared by the GEMV and dequantize kernels:
// per-quantization geometry and the in-register unpack of a lane's unit of
// packed weights. gfx950 (CDNA4) only.
//
// A "unit" is the slice of one row's packed weights that one lane consumes per
// step: one Q4_0 block (16 bytes, 32 weights), one Q5_0 block (20 bytes: the
// uint32 high-bit mask then 16 nibble bytes, 32 weights) or half a Q8_0 block
// (16 int8 bytes, 16 weights). Block layout and weight order follow the
// reference decode (quantization.py:34-47): in a Q4_0/Q5_0 block, byte j's low
// nibble is weight j and its high nibble weight j+16; Q5_0 weight j takes bit j
// of the little-endian mask as its fifth bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "svq_launch.h"

namespace svq {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int QT> struct QTraits;

// The GEMV turns every weight's unsigned code (nibble, 5-bit code or
// int8 + 128) into the fp16 *subnormal* with the same bit pattern, i.e.
// code * 2^-24, with one v_perm_b32 per pair of weights and no conversion
// instruction. Products with fp16 activations are exact in fp32, so a block's
// sum_j code_j * x_j is exact up to fp32 addition; the code offset is removed
// by adding offset * sum_j x_j (kSxScale folds the 2^-24 scaling in), and the
// result is rescaled once by kOutScale at the end.
template <> struct QTraits<4> {
  static constexpr int kBlockQ = 16;       // payload bytes per block
  static constexpr int kUnitBytes = 16;    // payload bytes per unit
  static constexpr int kUnitWeights = 32;  // weights per unit
  static constexpr int kUnitsPerBlock = 1;
  static constexpr int kWords = 4;         // dwords loaded per unit
  static constexpr float kSxScale = -0x1p-21f;  // -8 * 2^-24
  static constexpr float kOutScale = 0x1p24f;
};
template <> struct QTraits<5> {
  static constexpr int kBlockQ = 20;
  static constexpr int kUnitBytes = 20;
  static constexpr int kUnitWeights = 32;
  static constexpr int kUnitsPerBlock = 1;
  static constexpr int kWords = 5;
  // Codes are placed as 16 * code subnormals (see unpack_q5): -16 * 2^-20.
  static constexpr float kSxScale = -0x1p-16f;
  static constexpr float kOutScale = 0x1p20f;
};
template <> struct QTraits<8> {
  static constexpr int kBlockQ = 32;
  static constexpr int kUnitBytes = 16;
  static constexpr int kUnitWeights = 16;
  static constexpr int kUnitsPerBlock = 2;
  static constexpr int kWords = 4;
  static constexpr float kSxScale = -0x1p-17f;  // -128 * 2^-24
  static constexpr float kOutScale = 0x1p24f;
};

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a),
                                __builtin_bit_cast(h2_t, b), c, false);
}

// v_perm_b32: byte i of the result is byte sel[i] of the 8-byte value
// {hi, lo} (0-3 = lo, 4-7 = hi, 0x0c = zero byte).
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo,
                                         uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

constexpr uint32_t kSelB01 = 0x0c010c00u;   // {lo.b0, 0, lo.b1, 0}
constexpr uint32_t kSelB23 = 0x0c030c02u;   // {lo.b2, 0, lo.b3, 0}
constexpr uint32_t kSelB01H = 0x05010400u;  // {lo.b0, hi.b0, lo.b1, hi.b1}
constexpr uint32_t kSelB23H = 0x07030602u;  // {lo.b2, hi.b2, lo.b3, hi.b3}

// Four mask bits (n < 16) spread to bit 0 of each byte:
// n * 0x204081 = n + n<<7 + n<<14 + n<<21 puts bit i of n at bit 8i, with no
// overlapping terms.
__device__ __forceinline__ uint32_t spread4(uint32_t n) {
  return (n * 0x00204081u) & 0x01010101u;
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// Unpack one unit into fp16 pairs p[j] = (weight 2j, weight 2j+1) as
// subnormal codes. Q4_0 returns the low-nibble half (weights 0-15, codes
// 0..15) in p[0..7] and the high-nibble half (weights 16-31) in p[8..15] as
// 16 * code, so the caller scales the second half's sum by 1/16. Q5_0 returns
// all 32 as 16 * code (code = nibble | fifth bit << 4). Q8_0 returns the 16
// weights of a half block as int8 + 128.
template <int QT>
__device__ __forceinline__ void unpack(const uint32_t (&w)[QTraits<QT>::kWords],
                                       uint32_t (&p)[QTraits<QT>::kUnitWeights / 2]);

template <>
__device__ __forceinline__ void unpack<4>(const uint32_t (&w)[4],
                                          uint32_t (&p)[16]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = w[i] & 0x0f0f0f0fu;  // codes of weights 4i..4i+3
    const uint32_t hi = w[i] & 0xf0f0f0f0u;  // 16 * codes of 16+4i..16+4i+3
    p[2 * i] = perm(0u, lo, kSelB01);
    p[2 * i + 1] = perm(0u, lo, kSelB23);
    p[8 + 2 * i] = perm(0u, hi, kSelB01);
    p[8 + 2 * i + 1] = perm(0u, hi, kSelB23);
  }
}

// unpack<4> with both nibble halves as 16 * code, for dot products that sum
// the two halves together (offset term and output scale as for Q5_0).
__device__ __forceinline__ void unpack_q4_x16(const uint32_t (&w)[4], uint32_t (&p)[16]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = (w[i] << 4) & 0xf0f0f0f0u;  // 16 * codes of weights 4i..4i+3
    const uint32_t hi = w[i] & 0xf0f0f0f0u;         // 16 * codes of 16+4i..16+4i+3
    p[2 * i] = perm(0u, lo, kSelB01);
    p[2 * i + 1] = perm(0u, lo, kSelB23);
    p[8 + 2 * i] = perm(0u, hi, kSelB01);
    p[8 + 2 * i + 1] = perm(0u, hi, kSelB23);
  }
}

template <>
__device__ __forceinline__ void unpack<5>(const uint32_t (&w)[5],
                                          uint32_t (&p)[16]) {
  const uint32_t qh = w[0];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t v = w[1 + i];
    const uint32_t lo = (v << 4) & 0xf0f0f0f0u;  // 16 * low nibbles
    const uint32_t hi = v & 0xf0f0f0f0u;         // 16 * high nibbles
    const uint32_t blo = spread4((qh >> (4 * i)) & 15u);
    const uint32_t bhi = spread4((qh >> (16 + 4 * i)) & 15u);
    // Fifth bit as the high byte of each half: 16 * nibble + 256 * bit.
    p[2 * i] = perm(blo, lo, kSelB01H);
    p[2 * i + 1] = perm(blo, lo, kSelB23H);
    p[8 + 2 * i] = perm(bhi, hi, kSelB01H);
    p[8 + 2 * i + 1] = perm(bhi, hi, kSelB23H);
  }
}

// Q5_0 mask expansion through a 256-entry LDS table: entry b (8 bytes at
// byte offset 8 * b) holds {spread4(b & 15), spread4(b >> 4)}, the fifth bits
// of 8 consecutive weights as bytes. The table sits at LDS offset 0, so a
// lookup address is 8 * (mask byte): two instructions per 8 weights instead
// of six for the multiply-and-mask spread.
constexpr int kQ5TableBytes = 256 * 8;

__device__ __forceinline__ void build_q5_table(u32x2* table, int tid, int nthreads) {
  for (int b = tid; b < 256; b += nthreads) {
    u32x2 e;
    e.x = spread4((uint32_t)b & 15u);
    e.y = spread4((uint32_t)b >> 4);
    table[b] = e;
  }
}

// unpack<5> with the mask bits expanded by table lookups (same output).
__device__ __forceinline__ void unpack_q5_table(const uint32_t (&w)[5], uint32_t (&p)[16],
                                                const u32x2* table) {
  const uint32_t qh = w[0];
  const char* base = reinterpret_cast<const char*>(table);
  // Mask byte k, times 8 (the table stride), as a byte offset.
  const u32x2 b0 = *reinterpret_cast<const u32x2*>(base + 8u * (qh & 0xffu));
  const u32x2 b1 = *reinterpret_cast<const u32x2*>(base + 8u * ((qh >> 8) & 0xffu));
  const u32x2 b2 = *reinterpret_cast<const u32x2*>(base + 8u * ((qh >> 16) & 0xffu));
  const u32x2 b3 = *reinterpret_cast<const u32x2*>(base + 8u * (qh >> 24));
  const uint32_t blo[4] = {b0.x, b0.y, b1.x, b1.y};  // weights 0-15
  const uint32_t bhi[4] = {b2.x, b2.y, b3.x, b3.y};  // weights 16-31
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t v = w[1 + i];
    const uint32_t lo = (v << 4) & 0xf0f0f0f0u;
    const uint32_t hi = v & 0xf0f0f0f0u;
    p[2 * i] = perm(blo[i], lo, kSelB01H);
    p[2 * i + 1] = perm(blo[i], lo, kSelB23H);
    p[8 + 2 * i] = perm(bhi[i], hi, kSelB01H);
    p[8 + 2 * i + 1] = perm(bhi[i], hi, kSelB23H);
  }
}

template <>
__device__ __forceinline__ void unpack<8>(const uint32_t (&w)[4],
                                          uint32_t (&p)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t v = w[i] ^ 0x80808080u;  // int8 -> int8 + 128
    p[2 * i] = perm(0u, v, kSelB01);
    p[2 * i + 1] = perm(0u, v, kSelB23);
  }
}

// Dot product of one unpacked unit with its activations xv (fp16 pairs in
// natural order), started from `start` (the offset term). Result is in units
// of the code scaling (2^-24, or 2^-20 for Q5_0).
template <int QT>
__device__ __forceinline__ float unit_dot(const uint32_t (&p)[QTraits<QT>::kUnitWeights / 2],
                                          const uint32_t (&xv)[QTraits<QT>::kUnitWeights / 2],
                                          float start);

template <>
__device__ __forceinline__ float unit_dot<4>(const uint32_t (&p)[16],
                                             const uint32_t (&xv)[16],
                                             float start) {
  float lo = start, hi = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) lo = dot2(p[j], xv[j], lo);
#pragma unroll
  for (int j = 8; j < 16; ++j) hi = dot2(p[j], xv[j], hi);
  return __builtin_fmaf(hi, 0.0625f, lo);
}

template <>
__device__ __forceinline__ float unit_dot<5>(const uint32_t (&p)[16],
                                             const uint32_t (&xv)[16],
                                             float start) {
  // Two chains for latency; both halves share the 16 * code scaling.
  float a = start, b = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) a = dot2(p[j], xv[j], a);
#pragma unroll
  for (int j = 8; j < 16; ++j) b = dot2(p[j], xv[j], b);
  return a + b;
}

template <>
__device__ __forceinline__ float unit_dot<8>(const uint32_t (&p)[8],
                                             const uint32_t (&xv)[8],
                                             float start) {
  float a = start, b = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) a = dot2(p[j], xv[j], a);
#pragma unroll
  for (int j = 4; j < 8; ++j) b = dot2(p[j], xv[j], b);
  return a + b;
}

// Signed integer weights of one unit (for dequantization), exactly as the
// reference computes them (quantization.py:34-47).
template <int QT>
__device__ __forceinline__ void unit_codes(const uint32_t (&w)[QTraits<QT>::kWords],
                                           int (&v)[QTraits<QT>::kUnitWeights]);

template <>
__device__ __forceinline__ void unit_codes<4>(const uint32_t (&w)[4], int (&v)[32]) {
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const uint32_t byte = (w[j >> 2] >> (8 * (j & 3))) & 0xffu;
    v[j] = (int)(byte & 15u) - 8;
    v[j + 16] = (int)(byte >> 4) - 8;
  }
}

template <>
__device__ __forceinline__ void unit_codes<5>(const uint32_t (&w)[5], int (&v)[32]) {
  const uint32_t qh = w[0];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const uint32_t byte = (w[1 + (j >> 2)] >> (8 * (j & 3))) & 0xffu;
    v[j] = (int)((byte & 15u) | (((qh >> j) & 1u) << 4)) - 16;
    v[j + 16] = (int)((byte >> 4) | (((qh >> (j + 16)) & 1u) << 4)) - 16;
  }
}

template <>
__device__ __forceinline__ void unit_codes<8>(const uint32_t (&w)[4], int (&v)[16]) {
#pragma unroll
  for (int j = 0; j < 16; ++j)
    v[j] = (int)(int8_t)((w[j >> 2] >> (8 * (j & 3))) & 0xffu);
}

// Buffer resource over `bytes` bytes from the wave-uniform `base`: loads use
// 32-bit offsets (no per-lane 64-bit address arithmetic) and reads beyond
// `bytes` return zeros instead of touching memory. The last word is the gfx9
// family's raw-buffer format (32-bit data format, no swizzle).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base,
                                                           uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                           (int)bytes, 0x00020000);
}

// Cache policy of weight loads that stream whole 16-byte units: the
// non-temporal hint (the `nt` bit of the buffer load's cache-policy operand).
// Measured on row-contiguous 16-byte unit loads (Q4_0, Q8_0), whose every
// load instruction covers whole cache lines: 49152 x 4608 at M = 1, Q4_0
// 27.2 -> 24.5 us and Q8_0 46.0 -> 41.4 us. Loads that cover a line in
// parts across instructions (the 20-byte Q5_0 units, runs of blocks per
// lane) turn 1.3-1.7x slower with it, so those keep the default policy.
constexpr int kLoadNonTemporal = 2;

// Load one unit's dwords at byte offset `off` of a buffer resource, with
// cache policy AUX for the 16-byte part.
template <int QT, int AUX = 0>
__device__ __forceinline__ void load_unit_buf(__amdgpu_buffer_rsrc_t r,
                                              uint32_t off,
                                              uint32_t (&w)[QTraits<QT>::kWords]) {
  const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX);
  w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  if constexpr (QT == 5) w[4] = __builtin_amdgcn_raw_buffer_load_b32(r, off + 16, 0, 0);
}

// Load one unit's dwords. Q4_0/Q8_0 units are 16-byte aligned (one
// global_load_dwordx4); Q5_0 units are 20 bytes apart, i.e. dword aligned:
// one dwordx4 plus one dword.
template <int QT>
__device__ __forceinline__ void load_unit(const uint8_t* p,
                                          uint32_t (&w)[QTraits<QT>::kWords]) {
  if constexpr (QT == 5) {
    typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
    const u32x4a4 a = *reinterpret_cast<const u32x4a4*>(p);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = *reinterpret_cast<const uint32_t*>(p + 16);
  } else {
    const u32x4 a = *reinterpret_cast<const u32x4*>(p);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  }
}

}  // namespace svq

namespace svq {

// Sum of v over the G = 1 << lg_g consecutive lanes of a lane group, left in
// every lane of the group: DPP quad permutes and row mirrors within 16 lanes,
// then the gfx950 lane-swap instructions across 16- and 32-lane halves. No
// LDS traffic.
__device__ __forceinline__ float group_sum(float v, int lg_g) {
  auto dpp = [](float f, auto ctrl) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(
        __builtin_bit_cast(int, f), decltype(ctrl)::value, 0xf, 0xf, false));
  };
  if (lg_g >= 1) v += dpp(v, std::integral_constant<int, 0xb1>{});   // quad_perm [1,0,3,2]
  if (lg_g >= 2) v += dpp(v, std::integral_constant<int, 0x4e>{});   // quad_perm [2,3,0,1]
  if (lg_g >= 3) v += dpp(v, std::integral_constant<int, 0x141>{});  // row_half_mirror
  if (lg_g >= 4) v += dpp(v, std::integral_constant<int, 0x140>{});  // row_mirror
  if (lg_g >= 5) {
    const int i = __builtin_bit_cast(int, v);
    const auto r = __builtin_amdgcn_permlane16_swap(i, i, false, false);
    v = __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
  }
  if (lg_g >= 6) {
    const int i = __builtin_bit_cast(int, v);
    const auto r = __builtin_amdgcn_permlane32_swap(i, i, false, false);
    v = __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
  }
  return v;
}

// Staging of x[:, cu0 : cu0 + cun units] (fp16, all M rows) into LDS in
// piece-major order, xs[(m * P + p) * stride + u], followed by the per-unit,
// per-row offset term kSxScale * sum(x over the unit) in sxs[m * stride + u].
//
// Split in two so that a kernel can put other loads between them: begin()
// issues the global loads of the first SB pieces of every thread into
// registers; finish() writes them to LDS, stages any remaining pieces in
// batches of SB, computes the offset sums and ends with a barrier. Loads
// retire in issue order, so loads issued between begin() and finish() (the
// weight stream) do not delay the first LDS writes. Batch entries past the end
// re-write the last piece with the same data, so every loaded register is
// consumed on every path.
// SxMul multiplies the offset term: 16 for a kernel that places every Q4_0
// code as 16 * code (both nibble halves scaled alike).
template <int QT, int M, int THREADS, int SB, int SxMul = 1, bool LN = false>
struct XStager {
  using T = QTraits<QT>;
  static constexpr int P = T::kUnitWeights / 8;
  __amdgpu_buffer_rsrc_t xr;  // the M rows of x, fp16 [M, k]
  int k, cu0, cun, stride, per_row, total;
  float inv_row;  // 1 / per_row
  u32x4 v[SB];
  int dst[SB];
#if SVQ_TIMELINE
  // Timeline builds: this wave's stamp slots (null: no stamps).
  unsigned long long* stamps = nullptr;
  __device__ __forceinline__ void stamp(int slot) const {
    if (stamps && (threadIdx.x & 63) == 0) stamps[slot] = __builtin_amdgcn_s_memrealtime();
  }
#else
  __device__ __forceinline__ void stamp(int) const {}
#endif

  __device__ __forceinline__ XStager(const uint16_t* x_, int k_, int cu0_, int cun_, int stride_)
      : xr(make_rsrc(x_, (uint32_t)(M * k_) * 2u)), k(k_), cu0(cu0_), cun(cun_), stride(stride_),
        per_row(cun_ * P), total(M * cun_ * P),
        inv_row(__builtin_amdgcn_rcpf((float)(cun_ * P))) {}

  // Row of piece t (0 <= t < total): t / per_row from the reciprocal. Exact
  // for per_row <= 2^14 (x of a row fits in LDS): (t + 1/2) / per_row lies at
  // least 2^-15 from an integer, and the product's relative error is a few
  // 2^-24 on a quotient below 8.
  __device__ __forceinline__ int row_of(int t) const {
    return M == 1 ? 0 : (int)(((float)t + 0.5f) * inv_row);
  }

  __device__ __forceinline__ void load_batch(int base) {
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      int t = min(base + j * THREADS, total - 1);
      const int m = row_of(t);
      t -= m * per_row;
      const int u = t / P, pc = t - u * P;
      const uint32_t off = (uint32_t)(m * k + cu0 * T::kUnitWeights) * 2u + (uint32_t)t * 16u;
      v[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
      dst[j] = (m * P + pc) * stride + u;
    }
  }

  __device__ __forceinline__ void store_batch(u32x4* xs) {
#pragma unroll
    for (int j = 0; j < SB; ++j) xs[dst[j]] = v[j];
  }

  // LayerNorm of every staged row (LN kernels only; full rows only: cu0 == 0,
  // cun units = k). Its weight and bias pieces (8 columns each) are copied to LDS by the
  // buffer unit (loads with an LDS destination, no registers) in begin(),
  // before the x loads: wave w copies the 64-piece blocks w, w + W, ...
  // (W waves) of each array to lns[block * 64 ...] (weight) and
  // lns[ln_cols() + block * 64 ...] (bias). Vector loads retire in issue
  // order, so the wait for a wave's own x pieces in finish() also covers its
  // copies, and the barrier after the x stores makes every copy visible
  // before the normalization reads them; no wait on the loads a kernel issues
  // between begin() and finish() is involved.
  static constexpr int kWaves = THREADS / 64;
  const uint16_t* ln_w = nullptr;
  const uint16_t* ln_b = nullptr;
  float ln_eps = 0.f;
  __device__ __forceinline__ void set_layer_norm(const uint16_t* w, const uint16_t* b,
                                                 float eps) {
    ln_w = w;
    ln_b = b;
    ln_eps = eps;
  }
  __device__ __forceinline__ bool has_layer_norm() const { return ln_w || ln_b; }
  // Pieces per parameter array in LDS: k / 8 rounded up to whole 64-piece
  // blocks (the copy writes 64 pieces per instruction).
  __device__ __forceinline__ int ln_cols() const { return (k / 8 + 63) / 64 * 64; }

  __device__ __forceinline__ void begin(u32x4* lns = nullptr) {
    if (LN && has_layer_norm()) {
      const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, cols = k / 8;
      // A missing array is a zero-length range: its copy writes zeros.
      const __amdgpu_buffer_rsrc_t wr = make_rsrc(ln_w, ln_w ? (uint32_t)cols * 16u : 0u);
      const __amdgpu_buffer_rsrc_t br = make_rsrc(ln_b, ln_b ? (uint32_t)cols * 16u : 0u);
      for (int blk = wv; blk * 64 < cols; blk += kWaves) {
        const uint32_t off = (uint32_t)(blk * 64 + lane) * 16u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            wr, (__attribute__((address_space(3))) void*)(lns + blk * 64), 16, off, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            br, (__attribute__((address_space(3))) void*)(lns + ln_cols() + blk * 64), 16, off,
            0, 0, 0);
      }
    }
    load_batch(threadIdx.x);
  }

  // Sum of s[] over the workgroup, left in every thread (red: one float per
  // wave and row).
  __device__ __forceinline__ void block_sum(float (&s)[M], float (*red)[M]) const {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
    for (int mm = 0; mm < M; ++mm) {
      const float v = group_sum(s[mm], 6);
      if (lane == 0) red[wv][mm] = v;
    }
    __syncthreads();
#pragma unroll
    for (int mm = 0; mm < M; ++mm) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < THREADS / 64; ++w) v += red[w][mm];
      s[mm] = v;
    }
  }

  // torch.nn.LayerNorm over each row of the staged x, in place in LDS: mean
  // and biased variance in fp32 (two passes), then
  // fp16((x - mean) * rstd * weight + bias). Piece (m, pc, u) of the LDS
  // layout holds columns u * kUnitWeights + pc * 8 .. + 7 of row m.
  __device__ __forceinline__ void layer_norm(u32x4* xs, const u32x4* lns) {
    __shared__ float red1[THREADS / 64][M], red2[THREADS / 64][M];
    const uint32_t ones = 0x3c003c00u;
    float s[M], mean[M], rstd[M];
#pragma unroll
    for (int mm = 0; mm < M; ++mm) {
      s[mm] = 0.f;
#pragma unroll
      for (int pc = 0; pc < P; ++pc)
        for (int u = threadIdx.x; u < cun; u += THREADS) {
          const u32x4 w = xs[(mm * P + pc) * stride + u];
          s[mm] = dot2(w.w, ones, dot2(w.z, ones, dot2(w.y, ones, dot2(w.x, ones, s[mm]))));
        }
    }
    block_sum(s, red1);
#pragma unroll
    for (int mm = 0; mm < M; ++mm) {
      mean[mm] = s[mm] / (float)k;
      float q = 0.f;
#pragma unroll
      for (int pc = 0; pc < P; ++pc)
        for (int u = threadIdx.x; u < cun; u += THREADS) {
          const u32x4 w = xs[(mm * P + pc) * stride + u];
          const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const h2_t h = __builtin_bit_cast(h2_t, ww[i]);
            const float d0 = (float)h.x - mean[mm], d1 = (float)h.y - mean[mm];
            q = fmaf(d0, d0, fmaf(d1, d1, q));
          }
        }
      s[mm] = q;
    }
    block_sum(s, red2);
#pragma unroll
    for (int mm = 0; mm < M; ++mm) rstd[mm] = 1.0f / sqrtf(s[mm] / (float)k + ln_eps);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, cols = k / 8, bcol = ln_cols();
    const bool unit_w = ln_w == nullptr;
    for (int blk = wv; blk * 64 < cols; blk += kWaves) {
      const int c = blk * 64 + lane;
      if (c >= cols) continue;
      const int u = c / P, pc = c - u * P;
      const u32x4 g = lns[c], b = lns[bcol + c];
      const uint32_t gg[4] = {g.x, g.y, g.z, g.w}, bb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
      for (int mm = 0; mm < M; ++mm) {
        const int word = (mm * P + pc) * stride + u;
        const u32x4 w = xs[word];
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const h2_t h = __builtin_bit_cast(h2_t, ww[i]);
          const h2_t gh = __builtin_bit_cast(h2_t, gg[i]);
          const h2_t bh = __builtin_bit_cast(h2_t, bb[i]);
          const float g0 = unit_w ? 1.0f : (float)gh.x, g1 = unit_w ? 1.0f : (float)gh.y;
          h2_t r;
          r.x = (_Float16)fmaf(((float)h.x - mean[mm]) * rstd[mm], g0, (float)bh.x);
          r.y = (_Float16)fmaf(((float)h.y - mean[mm]) * rstd[mm], g1, (float)bh.y);
          o[i] = __builtin_bit_cast(uint32_t, r);
        }
        xs[word] = u32x4{o[0], o[1], o[2], o[3]};
      }
    }
    __syncthreads();
  }

  // The LayerNorm when the first batch holds every piece of x (total <=
  // SB * THREADS): statistics from the registers, then only the normalized
  // pieces are written to LDS. Two barriers fewer than layer_norm().
  __device__ __forceinline__ void layer_norm_registers(u32x4* xs, const u32x4* lns) {
    __shared__ float red1[THREADS / 64][M], red2[THREADS / 64][M];
    const uint32_t ones = 0x3c003c00u;
    int row[SB], col[SB];
    bool valid[SB];
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      const int t = threadIdx.x + j * THREADS;
      valid[j] = t < total;
      const int r = valid[j] ? t : 0, m = row_of(r);
      row[j] = m;
      col[j] = r - m * per_row;  // = u * P + pc: the piece's column / 8 (full rows)
    }
    float s[M], mean[M], rstd[M];
#pragma unroll
    for (int mm = 0; mm < M; ++mm) s[mm] = 0.f;
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      const u32x4 w = v[j];
      const float ps = dot2(w.w, ones, dot2(w.z, ones, dot2(w.y, ones, dot2(w.x, ones, 0.f))));
#pragma unroll
      for (int mm = 0; mm < M; ++mm) s[mm] += valid[j] && row[j] == mm ? ps : 0.f;
    }
    block_sum(s, red1);
    stamp(8);
#pragma unroll
    for (int mm = 0; mm < M; ++mm) {
      mean[mm] = s[mm] / (float)k;
      s[mm] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      float mu = mean[0];
#pragma unroll
      for (int mm = 1; mm < M; ++mm) mu = row[j] == mm ? mean[mm] : mu;
      const uint32_t ww[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
      float q = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const h2_t h = __builtin_bit_cast(h2_t, ww[i]);
        const float d0 = (float)h.x - mu, d1 = (float)h.y - mu;
        q = fmaf(d0, d0, fmaf(d1, d1, q));
      }
#pragma unroll
      for (int mm = 0; mm < M; ++mm) s[mm] += valid[j] && row[j] == mm ? q : 0.f;
    }
    block_sum(s, red2);
    stamp(9);
#pragma unroll
    for (int mm = 0; mm < M; ++mm) rstd[mm] = 1.0f / sqrtf(s[mm] / (float)k + ln_eps);
    const int bcol = ln_cols();
    const bool unit_w = ln_w == nullptr;
    // Every piece's parameters first (a piece past the end reads column 0's
    // and is not stored), so the LDS reads are in flight together rather than
    // one piece at a time behind a branch.
    u32x4 gp[SB], bp[SB];
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      gp[j] = lns[col[j]];
      bp[j] = lns[bcol + col[j]];
    }
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      float mu = mean[0], rs = rstd[0];
#pragma unroll
      for (int mm = 1; mm < M; ++mm) {
        mu = row[j] == mm ? mean[mm] : mu;
        rs = row[j] == mm ? rstd[mm] : rs;
      }
      const u32x4 g = gp[j], b = bp[j];
      const uint32_t ww[4] = {v[j].x, v[j].y, v[j].z, v[j].w}, gg[4] = {g.x, g.y, g.z, g.w},
                     bb[4] = {b.x, b.y, b.z, b.w};
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const h2_t h = __builtin_bit_cast(h2_t, ww[i]);
        const h2_t gh = __builtin_bit_cast(h2_t, gg[i]);
        const h2_t bh = __builtin_bit_cast(h2_t, bb[i]);
        const float g0 = unit_w ? 1.0f : (float)gh.x, g1 = unit_w ? 1.0f : (float)gh.y;
        h2_t r;
        r.x = (_Float16)fmaf(((float)h.x - mu) * rs, g0, (float)bh.x);
        r.y = (_Float16)fmaf(((float)h.y - mu) * rs, g1, (float)bh.y);
        o[i] = __builtin_bit_cast(uint32_t, r);
      }
      if (valid[j]) xs[dst[j]] = u32x4{o[0], o[1], o[2], o[3]};
    }
    __syncthreads();
    stamp(10);
  }

  // lns: the LDS that begin() filled with the LayerNorm parameters
  // (2 * ln_cols() pieces), used only when set_layer_norm() gave any.
  __device__ __forceinline__ void finish(u32x4* xs, float* sxs, u32x4* lns = nullptr) {
    if (LN && has_layer_norm() && total <= SB * THREADS) {
      layer_norm_registers(xs, lns);
    } else {
      store_batch(xs);
      for (int base = threadIdx.x + SB * THREADS; base < total; base += SB * THREADS) {
        load_batch(base);
        store_batch(xs);
      }
      __syncthreads();
      if (LN && has_layer_norm()) layer_norm(xs, lns);
    }
    const uint32_t ones = 0x3c003c00u;  // fp16 pair (1, 1)
    for (int t = threadIdx.x; t < M * cun; t += THREADS) {
      const int m = t / cun, u = t - m * cun;
      float sx = 0.f;
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const u32x4 w = xs[(m * P + p) * stride + u];
        sx = dot2(w.x, ones, sx);
        sx = dot2(w.y, ones, sx);
        sx = dot2(w.z, ones, sx);
        sx = dot2(w.w, ones, sx);
      }
      sxs[m * stride + u] = sx * (T::kSxScale * SxMul);
    }
    __syncthreads();
  }
};

template <int QT, int M, int THREADS>
__device__ __forceinline__ void stage_x(const uint16_t* __restrict__ x, int k,
                                        int cu0, int cun, int stride,
                                        u32x4* xs, float* sxs) {
  XStager<QT, M, THREADS, 4> st(x, k, cu0, cun, stride);
  st.begin();
  st.finish(xs, sxs);
}

// GELU with the tanh approximation (Hendrycks and Gimpel, 2016):
// 0.5 x (1 + tanh(sqrt(2 / pi) (x + 0.044715 x^3))), in fp32.
__device__ __forceinline__ float gelu_tanh(float x) {
  const float kSqrt2OverPi = 0.7978845608028654f;
  const float inner = kSqrt2OverPi * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}

// Store y[m, row] = v (the bias-added fp32 result) with the fused epilogue:
// fp32 output as is; fp16 output rounded, then GELU (rounded again), then
// the residual added (rounded again), each step as the separate fp16 torch op
// it replaces.
// store_y of element i with its residual already loaded (`res`, the fp16
// bits; unused without a residual or with fp32 output).
__device__ __forceinline__ void store_y_loaded(const GemvArgs& a, size_t i, float v,
                                               uint16_t res) {
  if (a.y_f32) {
    reinterpret_cast<float*>(a.y)[i] = v;
    return;
  }
  _Float16 t = (_Float16)v;
  if (a.act == 1) t = (_Float16)gelu_tanh((float)t);
  if (a.residual) t = (_Float16)(half_bits_to_float(res) + (float)t);
  reinterpret_cast<_Float16*>(a.y)[i] = t;
}

__device__ __forceinline__ void store_y(const GemvArgs& a, int m, int row, float v) {
  const size_t i = (size_t)m * a.n + row;
  if (a.y_f32) {
    reinterpret_cast<float*>(a.y)[i] = v;
    return;
  }
  _Float16 t = (_Float16)v;
  if (a.act == 1) t = (_Float16)gelu_tanh((float)t);
  if (a.residual) t = (_Float16)(half_bits_to_float(a.residual[i]) + (float)t);
  reinterpret_cast<_Float16*>(a.y)[i] = t;
}

}  // namespace svq
