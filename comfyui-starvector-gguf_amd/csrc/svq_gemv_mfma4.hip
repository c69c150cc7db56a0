// Streaming fused GGUF SoA dequantize + GEMV on the 4x4x4 matrix cores: the
// instantiations for M = 1..4 (one A half), the K-split finish kernel and the
// launch entry points. The kernel template is in svq_mfma4_kernel.h.
#include "svq_mfma4_kernel.h"

namespace svq {

namespace {

// Second kernel of the K split: y[m, row] = store(sum over the slices, in
// slice order, of the raw partial sums, times the code scaling, plus bias),
// with the same epilogue (rounding, GELU, residual) as the one-pass store.
// Every load of a thread (its slices, bias and residual) is issued before
// the first is used: one memory round trip instead of one per load.
__global__ __launch_bounds__(256) void split_finish_kernel(GemvArgs a, int m_rows,
                                                           float out_scale) {
  // The arguments the loads need, in scalar registers before the first
  // branch: one scalar memory round trip at entry. The pointers come back
  // from the asm as plain pointers; the casts restore the global address
  // space, so the loads stay global loads (not flat ones, which also count
  // against the LDS wait counter).
  typedef __attribute__((address_space(1))) const float gfloat;
  typedef __attribute__((address_space(1))) const uint16_t gu16;
  int n = a.n, slices = a.slices, y_f32 = a.y_f32;
  const float* partial_p = a.partial;
  const uint16_t* bias_pp = a.bias;
  const uint16_t* residual_p = a.residual;
  asm volatile("" : "+s"(n), "+s"(slices), "+s"(y_f32), "+s"(partial_p), "+s"(bias_pp),
                    "+s"(residual_p));
  gfloat* partial = (gfloat*)partial_p;
  gu16* bias_p = (gu16*)bias_pp;
  gu16* residual = (gu16*)residual_p;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= m_rows * n) return;
  const int m = i / n, row = i - m * n;
  // Every slot's load unconditionally (slots past `slices` re-read slice
  // 0), so all of them are in flight together: a load behind a branch is
  // waited for before the next branch.
  float p[kSplitMaxSlices];
#pragma unroll
  for (int sl = 0; sl < kSplitMaxSlices; ++sl)
    p[sl] = partial[((size_t)(sl < slices ? sl : 0) * m_rows + m) * n + row];
  const uint16_t bias = bias_p ? bias_p[row] : 0;
  const uint16_t res = residual && !y_f32 ? residual[i] : 0;
  float v = 0.f;
#pragma unroll
  for (int sl = 0; sl < kSplitMaxSlices; ++sl)
    if (sl < slices) v += p[sl];
  const float b = bias_p ? half_bits_to_float(bias) : 0.f;
  store_y_loaded(a, i, __builtin_fmaf(v, out_scale, b), res);
}

template <int QT>
hipError_t mfma4_dispatch_m(const GemvArgs& a, bool ln, int m, int rows, int groups, size_t lds,
                            hipStream_t stream, const void** fn) {
  switch (m) {
    case 1: return mfma4_dispatch_r<QT, 1>(a, ln, rows, groups, lds, stream, fn);
    case 2: return mfma4_dispatch_r<QT, 2>(a, ln, rows, groups, lds, stream, fn);
    case 3: return mfma4_dispatch_r<QT, 3>(a, ln, rows, groups, lds, stream, fn);
    case 4: return mfma4_dispatch_r<QT, 4>(a, ln, rows, groups, lds, stream, fn);
  }
  return hipErrorInvalidValue;
}

hipError_t mfma4_dispatch(const GemvArgs& a, bool ln, int qtype, int m, int rows, int groups,
                          size_t lds, hipStream_t stream, const void** fn) {
  if (m > 4) return mfma4_dispatch_wide(a, ln, qtype, m, rows, groups, lds, stream, fn);
  switch (qtype) {
    case 4: return mfma4_dispatch_m<4>(a, ln, m, rows, groups, lds, stream, fn);
    case 5: return mfma4_dispatch_m<5>(a, ln, m, rows, groups, lds, stream, fn);
    case 8: return mfma4_dispatch_m<8>(a, ln, m, rows, groups, lds, stream, fn);
  }
  return hipErrorInvalidValue;
}

}  // namespace

const void* mfma4_kernel(int qtype, int m, int rows, bool ln) {
  const void* fn = nullptr;
  GemvArgs unused{};
  (void)mfma4_dispatch(unused, ln, qtype, m, rows, 0, 0, nullptr, &fn);
  return fn;
}

size_t mfma4_lds_bytes(int qtype, int m, int k, int rows, int ksplit) {
  const size_t part = ksplit > 1 ? (size_t)2 * kStreamWavesPerGroup * (rows == 2 ? 2 : 1) * m * 4 * 4
                                 : 0;
  return stream_lds_bytes(qtype, m, k) + part;
}

// The kernel's work plan (GemvArgs::units .. lg_ksplit) for `groups`
// workgroups (a multiple of the K slices) of the `rows` variant.
GemvArgs plan_mfma4(const GemvArgs& in, int qtype, int rows, int groups) {
  GemvArgs a = in;
  const int sl = a.partial ? a.slices : 1;
  const int R = rows == 2 ? 2 : 1;
  const int U = rows == 3 ? (qtype == 8 ? 2 : 3) : 1;
  const int S = a.ksplit > 1 ? a.ksplit : 1;
  const int P = kStreamWavesPerGroup / S;
  const int G = groups / sl;
  a.units = (a.k / 32) * units_per_block(qtype) / sl;
  a.tiles = (a.n + 4 * R - 1) / (4 * R);
  a.tile_groups = (a.tiles + P - 1) / P;
  a.wave_major = S == 1 && a.tiles <= P * G;
  a.tiles_hi = (a.tile_groups + G - 1) / G;
  a.tiles_full = a.tile_groups - (a.tiles_hi - 1) * G;
  a.steps = (a.units + 16 * U - 1) / (16 * U);
  a.lg_ksplit = S == 4 ? 2 : S == 2 ? 1 : 0;
  // Q5_0 three-block lanes issue one ring step before x is staged when every
  // tile slot has at most one row tile (the kernel's SP variant).
  a.short_prologue = qtype == 5 && U == 3 && a.tiles <= P * G;
  return a;
}

hipError_t launch_gemv_mfma4(const GemvArgs& in, int qtype, int m, int rows, int groups,
                             hipStream_t stream) {
  const GemvArgs a = plan_mfma4(in, qtype, rows, groups);
  if (a.partial) {  // K slices: x staged per slice, then the slices added
    const hipError_t e = mfma4_dispatch(a, false, qtype, m, rows, groups,
                                        mfma4_lds_bytes(qtype, m, a.k / a.slices, rows, 1),
                                        stream, nullptr);
    if (e != hipSuccess) return e;
    const float out_scale = qtype == 8 ? Mfma4Traits<8>::kOutScale : Mfma4Traits<4>::kOutScale;
    const int total = m * a.n;
    hipLaunchKernelGGL(split_finish_kernel, dim3((total + 255) / 256), dim3(256), 0, stream, a,
                       m, out_scale);
    return hipGetLastError();
  }
  return mfma4_dispatch(a, a.ln_w || a.ln_b, qtype, m, rows, groups,
                        mfma4_lds_bytes(qtype, m, a.k, rows, a.ksplit) +
                            layer_norm_lds_bytes(a.k, a.ln_w || a.ln_b),
                        stream, nullptr);
}

#if SVQ_TIMELINE
namespace {
// A plain coalesced read of `bytes` (a multiple of 16): wave w of the grid
// reads the 1 KB pieces w, w + W, ... (64 lanes x 16 bytes each) and stamps
// its entry and end like the GEMV (slots 0 and 4).
__global__ __launch_bounds__(256) void timeline_read_kernel(const uint8_t* p, uint32_t bytes,
                                                            uint32_t* sink,
                                                            unsigned long long* stamps) {
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  const __amdgpu_buffer_rsrc_t r = make_rsrc(p, bytes);
  const uint32_t waves = gridDim.x * 4u, wave = blockIdx.x * 4u + (threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u, pieces = bytes / 1024u;
  uint32_t acc = 0;
  for (uint32_t i = wave; i < pieces; i += 8u * waves) {
    u32x4 v[8];
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) {
      const uint32_t pc = i + j * waves;
      v[j] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, pc < pieces ? pc * 1024u + lane * 16u
                                                                       : kOutOfRange, 0, 0));
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  }
  sink[blockIdx.x * 256u + threadIdx.x] = acc;
  if (lane == 0) {
    stamps[wave * kTimelineSlots] = t0;
    stamps[wave * kTimelineSlots + 4] = __builtin_amdgcn_s_memrealtime();
  }
}
}  // namespace

hipError_t launch_timeline_read(const void* p, uint32_t bytes, int groups, uint32_t* sink,
                                unsigned long long* stamps, hipStream_t stream) {
  hipLaunchKernelGGL(timeline_read_kernel, dim3(groups), dim3(256), 0, stream,
                     static_cast<const uint8_t*>(p), bytes, sink, stamps);
  return hipGetLastError();
}
#endif

}  // namespace svq
