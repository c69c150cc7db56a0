// Decode attention for one layer and one new token per row, fused with the
// rotary embedding of q and k and the write of the new key/value cache slot.
//
// Follows the decode branch of the reference blocks: StarCoder2
// (runtime_8b.py:38-55: rotate q and k, `index_copy_` of k and v into slot
// `position`, `baddbmm(bias, q, K^T, alpha = head_dim^-0.5)`, fp32 softmax,
// `bmm` with V) and the multi-query GPTBigCode block (runtime_1b.py:30-45:
// the same without the rotation, one key/value head). Query head h uses
// key/value head h / G, G = heads / kv_heads (contiguous groups, as the
// reference's `q.reshape(rows * kv_heads, G, head_dim)`).
//
// Numerics: a score is alpha * (q . k) + bias_j in fp32, rounded to fp16 as
// the reference's fp16 `baddbmm` output is; softmax and the weighted sum of V
// run in fp32 and the output is rounded to fp16 once. The reference also
// rounds the probabilities to fp16 before its `bmm`; this kernel keeps them in
// fp32 (relative difference below 2^-11 per term). The rotation is bit-exact
// with the reference's fp16 elementwise ops: fp16(fp16(x * cos) +
// fp16(rotate_half(x) * sin)), each product and the sum formed in fp32.
//
// Work split (flash decoding), two kernels:
// 1. Workgroup (c, r) takes cache chunk c (64 slots) of (row, kv head) r. Its
//    4 waves take 16 slots each; a 16-lane row of a wave holds one slot, lane
//    p of the row dims 8p..8p+7 of q, k and v. It writes the chunk's max
//    score, sum of exponentials and weighted sum of V per query head to the
//    workspace.
// 2. One workgroup per (row, query head) merges the chunks and writes the
//    output. The kernel boundary orders the two: no atomics, no fences.
#include <math.h>

#include "svq_device.h"
#include "svq_launch.h"

namespace svq {

namespace {

constexpr int kD = 128;                        // head dimension
constexpr int kWaves = 4;
constexpr int kIters = 4;                      // slots per 16-lane row
constexpr int kChunk = kWaves * 4 * kIters;    // slots per workgroup
constexpr uint32_t kOutOfRange = 0x80000000u;  // past every buffer range

__device__ __forceinline__ u32x4 load16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

__device__ __forceinline__ _Float16 lo_half(uint32_t v) {
  return __builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu));
}
__device__ __forceinline__ _Float16 hi_half(uint32_t v) {
  return __builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
}
__device__ __forceinline__ uint32_t pack_halves(_Float16 lo, _Float16 hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, lo) |
         ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
}

// One rotated element: fp16(fp16(x * c) + fp16(r * s)), r = -partner for the
// lower half of the head dims and +partner for the upper half. Contraction is
// off: a fused multiply-add would skip the rounding of the products.
__device__ __forceinline__ _Float16 rope1(_Float16 x, _Float16 partner, _Float16 c,
                                          _Float16 s, bool lower) {
#pragma clang fp contract(off)
  const float r = lower ? -(float)partner : (float)partner;
  const _Float16 a = (_Float16)((float)x * (float)c);
  const _Float16 b = (_Float16)(r * (float)s);
  return (_Float16)((float)a + (float)b);
}

__device__ __forceinline__ uint32_t rope2(uint32_t x, uint32_t partner, uint32_t c,
                                          uint32_t s, bool lower) {
  return pack_halves(rope1(lo_half(x), lo_half(partner), lo_half(c), lo_half(s), lower),
                     rope1(hi_half(x), hi_half(partner), hi_half(c), hi_half(s), lower));
}

__device__ __forceinline__ u32x4 rope8(u32x4 x, u32x4 partner, u32x4 c, u32x4 s, bool lower) {
  u32x4 r;
  r.x = rope2(x.x, partner.x, c.x, s.x, lower);
  r.y = rope2(x.y, partner.y, c.y, s.y, lower);
  r.z = rope2(x.z, partner.z, c.z, s.z, lower);
  r.w = rope2(x.w, partner.w, c.w, s.w, lower);
  return r;
}

__device__ __forceinline__ float dot8(u32x4 a, u32x4 b) {
  return dot2(a.w, b.w, dot2(a.z, b.z, dot2(a.y, b.y, dot2(a.x, b.x, 0.0f))));
}

// Combine v over the four 16-lane rows of a wave (same lane position in each
// row) with the gfx950 lane swaps; every lane receives the result.
template <bool kMax>
__device__ __forceinline__ float rows_reduce(float v) {
  int i = __builtin_bit_cast(int, v);
  auto r = __builtin_amdgcn_permlane16_swap(i, i, false, false);
  float a = __builtin_bit_cast(float, (int)r[0]), b = __builtin_bit_cast(float, (int)r[1]);
  v = kMax ? fmaxf(a, b) : a + b;
  i = __builtin_bit_cast(int, v);
  r = __builtin_amdgcn_permlane32_swap(i, i, false, false);
  a = __builtin_bit_cast(float, (int)r[0]);
  b = __builtin_bit_cast(float, (int)r[1]);
  return kMax ? fmaxf(a, b) : a + b;
}

template <int G>
__global__ __launch_bounds__(kWaves * 64) void decode_attention_kernel(AttnArgs a) {
  __shared__ float red[kWaves][G];
  __shared__ float accs[kWaves][G][kD + 4];

  const int c = blockIdx.x;
  const int rk = blockIdx.y;
  const int row = rk / a.kv_heads, kv = rk - row * a.kv_heads;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int p = lane & 15, sl = lane >> 4;
  const int64_t pos = *a.position;
  const int heads = a.kv_heads * G;

  // q of the G query heads of this kv head, and the new k and v, rotated.
  const uint16_t* qrow = a.qkv + (int64_t)row * a.qkv_stride;
  const bool rope = a.cos != nullptr;
  const bool lower = p < 8;
  const int partner = (8 * p + kD / 2) & (kD - 1);
  u32x4 cs = {0, 0, 0, 0}, sn = {0, 0, 0, 0};
  if (rope) {
    cs = load16(a.cos + 8 * p);
    sn = load16(a.sin + 8 * p);
  }
  u32x4 qv[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint16_t* qh = qrow + (kv * G + g) * kD;
    qv[g] = load16(qh + 8 * p);
    if (rope) qv[g] = rope8(qv[g], load16(qh + partner), cs, sn, lower);
  }
  const uint16_t* krow = qrow + (heads + kv) * kD;
  const uint16_t* vrow = qrow + (heads + a.kv_heads + kv) * kD;
  u32x4 knew = load16(krow + 8 * p);
  if (rope) knew = rope8(knew, load16(krow + partner), cs, sn, lower);
  const u32x4 vnew = load16(vrow + 8 * p);

  const int64_t slab = (int64_t)rk * a.capacity * kD;
  uint16_t* kslab = a.keys + slab;
  uint16_t* vslab = a.values + slab;
  const int c0 = c * kChunk;
  if (w == 0 && sl == 0 && pos >= c0 && pos < c0 + kChunk && pos < a.span) {
    *reinterpret_cast<u32x4*>(kslab + pos * kD + 8 * p) = knew;
    *reinterpret_cast<u32x4*>(vslab + pos * kD + 8 * p) = vnew;
  }

  // This lane's slots: c0 + w * 16 + it * 4 + sl. Masked slots (past the span
  // or with a -inf bias) and the new slot load nothing.
  const __amdgpu_buffer_rsrc_t kr = make_rsrc(kslab, (uint32_t)a.span * kD * 2);
  const __amdgpu_buffer_rsrc_t vr = make_rsrc(vslab, (uint32_t)a.span * kD * 2);
  u32x4 kk[kIters], vv[kIters];
  float bias[kIters];
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    const int j = c0 + w * 16 + it * 4 + sl;
    float b = -INFINITY;
    if (j < a.span) b = a.bias ? half_bits_to_float(a.bias[j]) : 0.0f;
    bias[it] = b;
    const bool load = b != -INFINITY && j != pos;
    const uint32_t off = load ? (uint32_t)j * kD * 2 + 16u * p : kOutOfRange;
    kk[it] = __builtin_amdgcn_raw_buffer_load_b128(kr, off, 0, 0);
    vv[it] = __builtin_amdgcn_raw_buffer_load_b128(vr, off, 0, 0);
  }
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    if (c0 + w * 16 + it * 4 + sl == pos) {
      kk[it] = knew;
      vv[it] = vnew;
    }
  }

  // Scores, rounded to fp16 as the reference's fp16 baddbmm output.
  float sc[kIters][G];
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float d = group_sum(dot8(qv[g], kk[it]), 4);
      sc[it][g] = bias[it] == -INFINITY ? -INFINITY
                                        : (float)(_Float16)(fmaf(a.scale, d, bias[it]));
    }
  }

  // Chunk max per head.
  float m[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float v = sc[0][g];
#pragma unroll
    for (int it = 1; it < kIters; ++it) v = fmaxf(v, sc[it][g]);
    m[g] = rows_reduce<true>(v);
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) red[w][g] = m[g];
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < G; ++g)
    m[g] = fmaxf(fmaxf(red[0][g], red[1][g]), fmaxf(red[2][g], red[3][g]));

  // Exponentials and the weighted sum of V over the chunk.
  float l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    l[g] = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = 0.0f;
  }
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    float vf[8];
    const uint32_t vw[4] = {vv[it].x, vv[it].y, vv[it].z, vv[it].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      vf[2 * i] = (float)lo_half(vw[i]);
      vf[2 * i + 1] = (float)hi_half(vw[i]);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float e = sc[it][g] == -INFINITY ? 0.0f : __expf(sc[it][g] - m[g]);
      l[g] += e;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[g][i] = fmaf(e, vf[i], acc[g][i]);
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    l[g] = rows_reduce<false>(l[g]);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = rows_reduce<false>(acc[g][i]);
  }
  if (sl == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int i = 0; i < 8; ++i) accs[w][g][8 * p + i] = acc[g][i];
      if (p == 0) accs[w][g][kD] = l[g];
    }
  }
  __syncthreads();

  // This chunk's partial per head: (max, sum of exponentials) and the
  // weighted sum of V.
  const int64_t head0 = (int64_t)rk * G;
  for (int e = tid; e < G * kD; e += kWaves * 64) {
    const int g = e / kD, i = e - g * kD;
    a.acc[((head0 + g) * a.nchunks + c) * kD + i] =
        accs[0][g][i] + accs[1][g][i] + accs[2][g][i] + accs[3][g][i];
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if (tid == g) {
      const float l_sum = accs[0][g][kD] + accs[1][g][kD] + accs[2][g][kD] + accs[3][g][kD];
      a.ml[(head0 + g) * a.nchunks + c] = make_float2(m[g], l_sum);
    }
  }
}

// Merge of the chunk partials of one query head (workgroup (row, h)): lane
// group s of 32 lanes takes chunks s, s + 8, ...; thread t of a group owns
// dims 4t..4t+3. All partial loads of a thread are independent and issued
// together; the chunk weights exp(m_c - max) come from wave 0 through LDS.
constexpr int kMergeSlices = 8;

__global__ __launch_bounds__(256) void merge_kernel(AttnMerge a) {
  extern __shared__ float wts[];  // [nchunks] chunk weights
  __shared__ float red[kMergeSlices][kD];
  __shared__ float total;
  const int head = blockIdx.x;  // row * heads + h == (row * kv_heads + kv) * G + g
  const int tid = threadIdx.x, d4 = (tid & 31) * 4, slice = tid >> 5;
  const int n = a.nchunks;
  const float2* ml = a.ml + (int64_t)head * n;
  const float* acc = a.acc + (int64_t)head * n * kD;

  if (tid < 64) {
    float mx = -INFINITY;
    for (int ch = tid; ch < n; ch += 64) mx = fmaxf(mx, ml[ch].x);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    float sum = 0.0f;
    for (int ch = tid; ch < n; ch += 64) {
      const float2 v = ml[ch];
      const float w = v.x == -INFINITY ? 0.0f : __expf(v.x - mx);
      wts[ch] = w;
      sum = fmaf(v.y, w, sum);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 64);
    if (tid == 0) total = sum;
  }
  __syncthreads();

  float o0 = 0.0f, o1 = 0.0f, o2 = 0.0f, o3 = 0.0f;
  for (int ch0 = slice; ch0 < n; ch0 += 4 * kMergeSlices) {
    float4 v[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int ch = ch0 + b * kMergeSlices;
      v[b] = ch < n ? *reinterpret_cast<const float4*>(acc + (int64_t)ch * kD + d4)
                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int ch = ch0 + b * kMergeSlices;
      const float w = ch < n ? wts[ch] : 0.0f;
      o0 = fmaf(v[b].x, w, o0);
      o1 = fmaf(v[b].y, w, o1);
      o2 = fmaf(v[b].z, w, o2);
      o3 = fmaf(v[b].w, w, o3);
    }
  }
  red[slice][d4] = o0;
  red[slice][d4 + 1] = o1;
  red[slice][d4 + 2] = o2;
  red[slice][d4 + 3] = o3;
  __syncthreads();
  if (tid < 32) {
    float r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float t = 0.0f;
#pragma unroll
      for (int sl = 0; sl < kMergeSlices; ++sl) t += red[sl][d4 + i];
      r[i] = t / total;
    }
    u32x2 packed;
    packed.x = pack_halves((_Float16)r[0], (_Float16)r[1]);
    packed.y = pack_halves((_Float16)r[2], (_Float16)r[3]);
    *reinterpret_cast<u32x2*>(a.out + (int64_t)head * kD + d4) = packed;
  }
}

template <int G>
hipError_t launch_g(const AttnArgs& a, int rows, hipStream_t stream) {
  const dim3 grid(a.nchunks, rows * a.kv_heads);
  hipLaunchKernelGGL(decode_attention_kernel<G>, grid, dim3(kWaves * 64), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

int attention_chunks(int span) { return (span + kChunk - 1) / kChunk; }

int64_t attention_ml_bytes(int rows, int heads, int span) {
  return ((int64_t)rows * heads * attention_chunks(span) * 8 + 255) / 256 * 256;
}

int64_t attention_workspace_bytes(int rows, int heads, int kv_heads, int span) {
  (void)kv_heads;
  return attention_ml_bytes(rows, heads, span) +
         (int64_t)rows * heads * attention_chunks(span) * kD * 4;
}

hipError_t launch_decode_attention(const AttnArgs& a, int rows, int group, hipStream_t stream) {
  const hipError_t e = launch_chunks(a, rows, group, stream);
  if (e != hipSuccess) return e;
  AttnMerge m{a.ml, a.acc, a.out, a.nchunks};
  hipLaunchKernelGGL(merge_kernel, dim3(rows * a.kv_heads * group), dim3(256),
                     a.nchunks * sizeof(float), stream, m);
  return hipGetLastError();
}

hipError_t launch_chunks(const AttnArgs& a, int rows, int group, hipStream_t stream) {
  switch (group) {
    case 1: return launch_g<1>(a, rows, stream);
    case 2: return launch_g<2>(a, rows, stream);
    case 3: return launch_g<3>(a, rows, stream);
    case 4: return launch_g<4>(a, rows, stream);
    case 5: return launch_g<5>(a, rows, stream);
    case 6: return launch_g<6>(a, rows, stream);
    case 7: return launch_g<7>(a, rows, stream);
    case 8: return launch_g<8>(a, rows, stream);
    case 9: return launch_g<9>(a, rows, stream);
    case 10: return launch_g<10>(a, rows, stream);
    case 11: return launch_g<11>(a, rows, stream);
    case 12: return launch_g<12>(a, rows, stream);
    case 13: return launch_g<13>(a, rows, stream);
    case 14: return launch_g<14>(a, rows, stream);
    case 15: return launch_g<15>(a, rows, stream);
    case 16: return launch_g<16>(a, rows, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace svq
