// SoA dequantization for gfx950: every weight is the exact fp32 product of
// its signed integer code and its block's fp16 scale, then rounded to the
// output type, as `dequantize_soa` computes it (quantization.py:93-105).
// One thread decodes a quarter block (8 weights) and writes them as one
// 16-byte store (fp16 / bf16) or two (fp32), so a wave's stores are
// contiguous. The row-gather variant (one thread per unit) serves
// `GGUFEmbedding.forward` (quantization.py:421-446) without index_select
// copies.
#include "svq_device.h"
#include "svq_launch.h"

namespace svq {

constexpr int kDqThreads = 256;

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t b = __builtin_bit_cast(uint32_t, f);
  if ((b & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;  // NaN, as torch
  b += 0x7fffu + ((b >> 16) & 1u);
  return (uint16_t)(b >> 16);
}

template <int OUT, int NV>
__device__ __forceinline__ void store_values(void* out, int64_t first,
                                             const float (&v)[NV]) {
  if constexpr (OUT == kOutF32) {
    u32x4* o = reinterpret_cast<u32x4*>(reinterpret_cast<float*>(out) + first);
#pragma unroll
    for (int i = 0; i < NV / 4; ++i)
      o[i] = u32x4{__builtin_bit_cast(uint32_t, v[4 * i]),
                   __builtin_bit_cast(uint32_t, v[4 * i + 1]),
                   __builtin_bit_cast(uint32_t, v[4 * i + 2]),
                   __builtin_bit_cast(uint32_t, v[4 * i + 3])};
  } else {
    uint16_t h[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if constexpr (OUT == kOutF16) {
        // The backend fuses product + conversion into v_fma_mixlo_f16 with a
        // +0 addend, which turns a -0 product into +0; the fp16 result always
        // carries the fp32 value's sign, so restore it from the fp32 bits.
        const uint32_t sign = (__builtin_bit_cast(uint32_t, v[i]) >> 16) & 0x8000u;
        h[i] = __builtin_bit_cast(uint16_t, (_Float16)v[i]) | (uint16_t)sign;
      } else {
        h[i] = f32_to_bf16_rne(v[i]);
      }
    }
    u32x4* o = reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(out) + first);
#pragma unroll
    for (int i = 0; i < NV / 8; ++i)
      o[i] = u32x4{h[8 * i] | ((uint32_t)h[8 * i + 1] << 16),
                   h[8 * i + 2] | ((uint32_t)h[8 * i + 3] << 16),
                   h[8 * i + 4] | ((uint32_t)h[8 * i + 5] << 16),
                   h[8 * i + 6] | ((uint32_t)h[8 * i + 7] << 16)};
  }
}

// Decode unit `unit` (global unit index) into fp32 values.
template <int QT>
__device__ __forceinline__ void decode_unit(const uint8_t* q, const uint16_t* s,
                                            int64_t unit,
                                            float (&v)[QTraits<QT>::kUnitWeights]) {
  using T = QTraits<QT>;
  uint32_t w[T::kWords];
  load_unit<QT>(q + unit * T::kUnitBytes, w);
  const float d = half_bits_to_float(s[unit / T::kUnitsPerBlock]);
  int c[T::kUnitWeights];
  unit_codes<QT>(w, c);
#pragma unroll
  for (int j = 0; j < T::kUnitWeights; ++j) v[j] = (float)c[j] * d;
}

// Codes of weights 8p .. 8p + 7 of block b (piece p = 0..3 of its 32).
// Q4_0 / Q5_0: weight j < 16 is the low nibble of payload byte j, weight
// j >= 16 the high nibble of byte j - 16; Q5_0 adds bit j of its qh word as
// bit 4. Q8_0: byte j as int8.
template <int QT>
__device__ __forceinline__ void decode_piece(const uint8_t* q, int64_t b, int p, int (&c)[8]) {
  uint32_t lo, hi;
  uint32_t qh = 0;
  if constexpr (QT == 4) {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(q + b * 16 + (p & 1) * 8);
    lo = w[0];
    hi = w[1];
  } else if constexpr (QT == 5) {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(q + b * 20);
    qh = w[0];
    lo = w[1 + (p & 1) * 2];
    hi = w[2 + (p & 1) * 2];
  } else {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(q + b * 32 + p * 8);
    lo = w[0];
    hi = w[1];
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t byte = ((i < 4 ? lo : hi) >> (8 * (i & 3))) & 0xffu;
    if constexpr (QT == 8) {
      c[i] = (int)(int8_t)byte;
    } else {
      const int nib = (int)((byte >> ((p >> 1) * 4)) & 15u);
      if constexpr (QT == 4) c[i] = nib - 8;
      else c[i] = (nib | (int)((qh >> (8 * p + i)) & 1u) << 4) - 16;
    }
  }
}

// One thread per 8 weights (a quarter block): a wave's stores cover
// contiguous output (1 KB at fp16).
template <int QT, int OUT>
__global__ __launch_bounds__(kDqThreads) void dequant_kernel(
    const uint8_t* __restrict__ q, const uint16_t* __restrict__ s,
    void* __restrict__ out, int64_t npieces) {
  const int64_t t = (int64_t)blockIdx.x * kDqThreads + threadIdx.x;
  if (t >= npieces) return;
  const int64_t b = t >> 2;
  const int p = (int)(t & 3);
  int c[8];
  decode_piece<QT>(q, b, p, c);
  const float d = half_bits_to_float(s[b]);
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = (float)c[j] * d;
  store_values<OUT>(out, t * 8, v);
}

template <int QT, int OUT>
__global__ __launch_bounds__(kDqThreads) void dequant_rows_kernel(
    const uint8_t* __restrict__ q, const uint16_t* __restrict__ s,
    const int64_t* __restrict__ ids, int64_t nids, int64_t nrows,
    int units_per_row, void* __restrict__ out) {
  using T = QTraits<QT>;
  const int64_t t = (int64_t)blockIdx.x * kDqThreads + threadIdx.x;
  if (t >= nids * units_per_row) return;
  const int64_t i = t / units_per_row;
  const int64_t ur = t - i * units_per_row;
  const int64_t id = ids[i];
  float v[T::kUnitWeights];
  if (id < 0 || id >= nrows) {
#pragma unroll
    for (int j = 0; j < T::kUnitWeights; ++j) v[j] = __builtin_nanf("");
  } else {
    decode_unit<QT>(q, s, id * units_per_row + ur, v);
  }
  store_values<OUT>(out, t * T::kUnitWeights, v);
}

template <int QT, int OUT>
static hipError_t dq(const uint8_t* q, const uint16_t* s, void* out,
                     int64_t nblocks, hipStream_t stream) {
  const int64_t npieces = nblocks * 4;
  const int64_t groups = (npieces + kDqThreads - 1) / kDqThreads;
  hipLaunchKernelGGL((dequant_kernel<QT, OUT>), dim3((unsigned)groups),
                     dim3(kDqThreads), 0, stream, q, s, out, npieces);
  return hipGetLastError();
}

template <int QT, int OUT>
static hipError_t dq_rows(const uint8_t* q, const uint16_t* s,
                          const int64_t* ids, int64_t nids, int64_t nrows,
                          int k, void* out, hipStream_t stream) {
  const int upr = (k / 32) * QTraits<QT>::kUnitsPerBlock;
  const int64_t total = nids * upr;
  const int64_t groups = (total + kDqThreads - 1) / kDqThreads;
  hipLaunchKernelGGL((dequant_rows_kernel<QT, OUT>), dim3((unsigned)groups),
                     dim3(kDqThreads), 0, stream, q, s, ids, nids, nrows, upr,
                     out);
  return hipGetLastError();
}

template <int QT>
static hipError_t dq_q(const uint8_t* q, const uint16_t* s, void* out,
                       int64_t nblocks, int out_dtype, hipStream_t stream) {
  switch (out_dtype) {
    case kOutF16: return dq<QT, kOutF16>(q, s, out, nblocks, stream);
    case kOutF32: return dq<QT, kOutF32>(q, s, out, nblocks, stream);
    case kOutBF16: return dq<QT, kOutBF16>(q, s, out, nblocks, stream);
  }
  return hipErrorInvalidValue;
}

template <int QT>
static hipError_t dq_rows_q(const uint8_t* q, const uint16_t* s,
                            const int64_t* ids, int64_t nids, int64_t nrows,
                            int k, void* out, int out_dtype,
                            hipStream_t stream) {
  switch (out_dtype) {
    case kOutF16: return dq_rows<QT, kOutF16>(q, s, ids, nids, nrows, k, out, stream);
    case kOutF32: return dq_rows<QT, kOutF32>(q, s, ids, nids, nrows, k, out, stream);
    case kOutBF16: return dq_rows<QT, kOutBF16>(q, s, ids, nids, nrows, k, out, stream);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_dequant(const uint8_t* q, const uint16_t* s, void* out,
                          int64_t nblocks, int qtype, int out_dtype,
                          hipStream_t stream) {
  switch (qtype) {
    case 4: return dq_q<4>(q, s, out, nblocks, out_dtype, stream);
    case 5: return dq_q<5>(q, s, out, nblocks, out_dtype, stream);
    case 8: return dq_q<8>(q, s, out, nblocks, out_dtype, stream);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_dequant_rows(const uint8_t* q, const uint16_t* s,
                               const int64_t* ids, int64_t nids, int64_t nrows,
                               int k, void* out, int qtype, int out_dtype,
                               hipStream_t stream) {
  switch (qtype) {
    case 4: return dq_rows_q<4>(q, s, ids, nids, nrows, k, out, out_dtype, stream);
    case 5: return dq_rows_q<5>(q, s, ids, nids, nrows, k, out, out_dtype, stream);
    case 8: return dq_rows_q<8>(q, s, ids, nids, nrows, k, out, out_dtype, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace svq
