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
// 1. Workgroup (c, r) takes cache chunk c (kChunk slots) of (row, kv head) r;
//    each of its kWaves waves computes the scores and the weighted V sums of 32
//    slots on the matrix cores (see decode_attention_kernel). It writes the
//    chunk's max score, sum of exponentials and weighted sum of V per query
//    head to the workspace.
// 2. One workgroup per (row, query head) merges the chunks and writes the
//    output. The kernel boundary orders the two: no atomics, no fences.
#include <math.h>

#include "svq_device.h"
#include "svq_launch.h"

namespace svq {

namespace {

constexpr int kD = 128;                        // head dimension
// Two waves (64-slot chunks): twice the workgroups of four-wave chunks for
// the same span (208 instead of 104 at beam 2, 4 kv heads, span 1537), with a
// shorter cross-wave reduction and twice the partials to merge. Measured in
// one process against four waves: 8B beam-2 decode 517 -> 524 steps/s,
// GPTBigCode-1B 1003 -> 1019; one wave (32-slot chunks): 510 and 997;
// three waves: 520 and 1001.
constexpr int kWaves = 2;
constexpr int kChunk = kWaves * 32;            // slots per workgroup (32 per wave)
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
// lower half of the head dims and +partner for the upper half. In fp16
// arithmetic: an fp16 product or sum is the correctly rounded exact result,
// which is what the reference's ops give (each formed exactly in fp32 -- the
// product always, the sum whenever rounding can matter -- then rounded).
// Contraction is off: a fused multiply-add would skip the product rounding.
__device__ __forceinline__ _Float16 rope1(_Float16 x, _Float16 partner, _Float16 c,
                                          _Float16 s, bool lower) {
#pragma clang fp contract(off)
  // Sign flip on the bits: exactly torch's negation, -0 for +0 included.
  const _Float16 r = __builtin_bit_cast(
      _Float16, (uint16_t)(__builtin_bit_cast(uint16_t, partner) ^ (lower ? 0x8000u : 0u)));
  const _Float16 a = x * c;
  const _Float16 b = r * s;
  return a + b;
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

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4_t mfma16x16x32(u32x4 a, u32x4 b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, a),
                                                __builtin_bit_cast(h8_t, b), c, 0, 0, 0);
}

// Chunk kernel. Wave w takes the 32 slots s0 = c0 + 32w .. s0 + 31 as two
// 16-slot tiles. Lane (n = lane % 16, g = lane / 16):
// * S = K Q^T on v_mfma_f32_16x16x32_f16, four k-steps of 32 dims: A = K
//   (row n = slot, k-slots = dims 32 ks + 8g .. + 7), B = Q^T (column n =
//   query head n of the group, same dims). D gives the lane head n and
//   slots 4g + i, i < 4, of each tile.
// * O = P V on the same instruction, eight 16-dim tiles: A = P (row n = head,
//   k-slot (g, e) = slot 4g + e of tile 0 for e < 4, of tile 1 for e >= 4:
//   exactly the scores the lane holds), B = V read back from LDS at the same
//   slots (column n = dim). D gives the lane dim 16dt + n of heads 4g + i.
// Heads n >= G compute on zero queries and are never stored.
template <int G>
__global__ __launch_bounds__(kWaves * 64) void decode_attention_kernel(AttnArgs a) {
  constexpr int kVRow = kD / 8 + 1;  // u32x4 per staged V row (one of padding)
  constexpr int kVBytes = kWaves * 32 * kVRow * 16;
  constexpr int kOBytes = kWaves * 16 * (kD + 4) * 4;
  __shared__ __attribute__((aligned(16))) unsigned char smem[kVBytes > kOBytes ? kVBytes : kOBytes];
  __shared__ float red[kWaves][16], lsum[kWaves][16];
  u32x4* vst = reinterpret_cast<u32x4*>(smem);  // [wave][32 slots][kVRow]
  float* ost = reinterpret_cast<float*>(smem);  // [wave][16 heads][kD + 4]

  const int c = blockIdx.x;
  const int rk = blockIdx.y;
  const int row = rk / a.kv_heads, kv = rk - row * a.kv_heads;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int64_t pos = *a.position;
  const int heads = a.kv_heads * G;
  const bool rope = a.cos != nullptr;

  // The loads go out in the order their data is needed, before any of it is
  // used (vector loads retire in issue order): q, the new key and value, the
  // rotation tables, then the chunk's keys and values. The rotations then
  // wait only for the first group, while the chunk loads are in flight.
  // Q^T (B of the score MFMAs): query head kv * G + n, zero for n >= G.
  const uint16_t* qrow = a.qkv + (int64_t)row * a.qkv_stride;
  u32x4 qb[4];
  const uint16_t* qh = qrow + (kv * G + (n < G ? n : 0)) * kD;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) qb[ks] = load16(qh + 32 * ks + 8 * g);
  // The new key (rotated below) and value at this lane's dims.
  u32x4 kn[4], vn[4];
  const uint16_t* krow = qrow + (heads + kv) * kD;
  const uint16_t* vrow = qrow + (heads + a.kv_heads + kv) * kD;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    kn[ks] = load16(krow + 32 * ks + 8 * g);
    vn[ks] = load16(vrow + 32 * ks + 8 * g);
  }
  // Rotation tables at the lane's dims 32 ks + 8g.
  u32x4 cs[4], sn[4];
  if (rope) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      cs[ks] = load16(a.cos + 32 * ks + 8 * g);
      sn[ks] = load16(a.sin + 32 * ks + 8 * g);
    }
  }

  const int64_t slab = (int64_t)rk * a.capacity * kD;
  uint16_t* kslab = a.keys + slab;
  uint16_t* vslab = a.values + slab;
  const int c0 = c * kChunk, s0 = c0 + 32 * w;
  const __amdgpu_buffer_rsrc_t kr = make_rsrc(kslab, (uint32_t)a.span * kD * 2);
  const __amdgpu_buffer_rsrc_t vr = make_rsrc(vslab, (uint32_t)a.span * kD * 2);

  // Bias of the lane's two key/value slots s0 + 16t + n (bkv) and of its
  // eight score slots s0 + 16t + 4g + i (bsc); -inf past the span and, with
  // a window, outside (position - window, position] (the decode step's
  // causal sliding-window mask, runtime_8b.py:103-105).
  auto hidden = [&](int j) { return a.window > 0 && (j > pos || j <= pos - a.window); };
  float bkv[2], bsc[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int j = s0 + 16 * t + n;
    bkv[t] = j >= a.span || hidden(j) ? -INFINITY
             : a.bias               ? half_bits_to_float(a.bias[j])
                                    : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int js = s0 + 16 * t + 4 * g + i;
      bsc[t][i] = js >= a.span || hidden(js) ? -INFINITY
                  : a.bias                   ? half_bits_to_float(a.bias[js])
                                             : 0.0f;
    }
  }

  // K (A of the score MFMAs) and V (staged to LDS) of slot s0 + 16t + n.
  // Slots before the position (every slot of the span without a bias) are
  // loaded without waiting for their bias; slots past the position, which a
  // decode step's bias masks, are loaded below only if their bias does not.
  // The new slot takes kn / vn and is written to the cache.
  u32x4 ka[2][4], va[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int j = s0 + 16 * t + n;
    const bool load = j < a.span && j != pos && !hidden(j) && (a.bias == nullptr || j < pos);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const uint32_t off = load ? (uint32_t)j * kD * 2 + (32u * ks + 8u * g) * 2 : kOutOfRange;
      ka[t][ks] = __builtin_amdgcn_raw_buffer_load_b128(kr, off, 0, 0);
      va[t][ks] = __builtin_amdgcn_raw_buffer_load_b128(vr, off, 0, 0);
    }
  }
  if (a.bias) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int j = s0 + 16 * t + n;
      if (j > pos && bkv[t] != -INFINITY) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const uint32_t off = (uint32_t)j * kD * 2 + (32u * ks + 8u * g) * 2;
          ka[t][ks] = __builtin_amdgcn_raw_buffer_load_b128(kr, off, 0, 0);
          va[t][ks] = __builtin_amdgcn_raw_buffer_load_b128(vr, off, 0, 0);
        }
      }
    }
  }

  // Rotation of a lane's 4 pieces (dims 32 ks + 8g): the partner of piece ks
  // is piece ks ^ 2 (dims + 64 mod 128); the lower half of the dims is ks < 2.
  auto rotate4 = [&](u32x4 (&v)[4]) {
    if (!rope) return;
    u32x4 r[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) r[ks] = rope8(v[ks], v[ks ^ 2], cs[ks], sn[ks], ks < 2);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) v[ks] = r[ks];
  };
  rotate4(qb);
  if (n >= G) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qb[ks] = u32x4{0, 0, 0, 0};
  }
  rotate4(kn);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int j = s0 + 16 * t + n;
    if (j == pos && pos < a.span) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        ka[t][ks] = kn[ks];
        va[t][ks] = vn[ks];
        *reinterpret_cast<u32x4*>(kslab + pos * kD + 32 * ks + 8 * g) = kn[ks];
        *reinterpret_cast<u32x4*>(vslab + pos * kD + 32 * ks + 8 * g) = vn[ks];
      }
    }
    if (bkv[t] == -INFINITY) {  // masked: its probability is 0, its V must be finite
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) va[t][ks] = u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) vst[(w * 32 + 16 * t + n) * kVRow + 4 * ks + g] = va[t][ks];
  }

  // Scores of head n at slots 4g + i of each tile, rounded to fp16 as the
  // reference's fp16 baddbmm output.
  float sc[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    f4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) d = mfma16x16x32(ka[t][ks], qb[ks], d);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float b = bsc[t][i];
      sc[t][i] = b == -INFINITY ? -INFINITY : (float)(_Float16)(fmaf(a.scale, d[i], b));
    }
  }

  // Chunk max per head: the lane's 8 slots, the 4 lane groups, the waves.
  float m = sc[0][0];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) m = fmaxf(m, sc[t][i]);
  m = rows_reduce<true>(m);
  if (g == 0) red[w][n] = m;
  __syncthreads();  // also orders the V staging before the reads below
  m = red[0][n];
#pragma unroll
  for (int ww = 1; ww < kWaves; ++ww) m = fmaxf(m, red[ww][n]);

  // P in fp16 (A of the PV MFMAs) and its fp32 sum.
  float l = 0.f;
  uint32_t pa[4];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    float e[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      e[i] = sc[t][i] == -INFINITY ? 0.0f : __expf(sc[t][i] - m);
      l += e[i];
    }
    pa[2 * t] = pack_halves((_Float16)e[0], (_Float16)e[1]);
    pa[2 * t + 1] = pack_halves((_Float16)e[2], (_Float16)e[3]);
  }
  l = rows_reduce<false>(l);
  if (g == 0) lsum[w][n] = l;
  const u32x4 pav = u32x4{pa[0], pa[1], pa[2], pa[3]};

  // O = P V per 16-dim tile; B gathers V[slot 4g + e (tile 0) / 16 + 4g + e - 4
  // (tile 1)][16 dt + n] from the wave's staged rows.
  const uint16_t* vw = reinterpret_cast<const uint16_t*>(vst + w * 32 * kVRow);
  f4_t o[kD / 16];
#pragma unroll
  for (int dt = 0; dt < kD / 16; ++dt) {
    const int dim = 16 * dt + n;
    uint32_t bv[4];
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      const int sa = (e2 < 2 ? 4 * g + 2 * e2 : 16 + 4 * g + 2 * (e2 - 2));
      const uint16_t lo = vw[sa * kVRow * 8 + dim], hi = vw[(sa + 1) * kVRow * 8 + dim];
      bv[e2] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
    o[dt] = mfma16x16x32(pav, u32x4{bv[0], bv[1], bv[2], bv[3]}, f4_t{0.f, 0.f, 0.f, 0.f});
  }
  __syncthreads();  // the V staging area becomes the O staging area

  // Sum of the waves' O, then this chunk's partial per head < G:
  // (max, sum of exponentials) and the weighted sum of V.
#pragma unroll
  for (int dt = 0; dt < kD / 16; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) ost[(w * 16 + 4 * g + i) * (kD + 4) + 16 * dt + n] = o[dt][i];
  __syncthreads();
  const int64_t head0 = (int64_t)rk * G;
  for (int e = tid; e < G * kD; e += kWaves * 64) {
    const int h = e / kD, d = e - h * kD;
    float v = 0.f;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) v += ost[(ww * 16 + h) * (kD + 4) + d];
    a.acc[((head0 + h) * a.nchunks + c) * kD + d] = v;
  }
  // Thread tid < G holds head n = tid's chunk max in m.
  if (tid < G) {
    float ls = lsum[0][tid];
#pragma unroll
    for (int ww = 1; ww < kWaves; ++ww) ls += lsum[ww][tid];
    a.ml[(head0 + tid) * a.nchunks + c] = make_float2(m, ls);
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

  // The first batch of partial loads goes out before the chunk weights are
  // known: both then take one round trip.
  float4 v[4];
  auto load_batch = [&](int ch0) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int ch = ch0 + b * kMergeSlices;
      v[b] = ch < n ? *reinterpret_cast<const float4*>(acc + (int64_t)ch * kD + d4)
                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  };
  load_batch(slice);

  if (tid < 64) {
    float mx = -INFINITY;
    for (int ch = tid; ch < n; ch += 64) mx = fmaxf(mx, ml[ch].x);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    float sum = 0.0f;
    for (int ch = tid; ch < n; ch += 64) {
      const float2 c = ml[ch];
      const float w = c.x == -INFINITY ? 0.0f : __expf(c.x - mx);
      wts[ch] = w;
      sum = fmaf(c.y, w, sum);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 64);
    if (tid == 0) total = sum;
  }
  __syncthreads();

  float o0 = 0.0f, o1 = 0.0f, o2 = 0.0f, o3 = 0.0f;
  for (int ch0 = slice;;) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int ch = ch0 + b * kMergeSlices;
      const float w = ch < n ? wts[ch] : 0.0f;
      o0 = fmaf(v[b].x, w, o0);
      o1 = fmaf(v[b].y, w, o1);
      o2 = fmaf(v[b].z, w, o2);
      o3 = fmaf(v[b].w, w, o3);
    }
    ch0 += 4 * kMergeSlices;
    if (ch0 >= n) break;
    load_batch(ch0);
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

// Beam reorder (the cache copies of runtime_shared.py:388-394): every row r
// whose parent p = parents[r] differs from r takes the first `length` slots
// of each (plane, head) of row p. A thread owns four 16-byte piece
// positions (256 apart) of one (plane, head) and moves them for every row,
// reading all sources before it writes, so rows that exchange caches need no
// staging copy. A parent outside [0, rows) leaves its row as it is.
constexpr int kReorderMaxRows = 8;
constexpr int kReorderPieces = 4;  // 16-byte pieces per thread (256 threads apart)

__global__ __launch_bounds__(256) void cache_reorder_kernel(ReorderArgs a) {
  const int64_t pieces = a.length * (kD / 8);  // 16-byte pieces per (plane, row, head)
  const int64_t e0 = (int64_t)blockIdx.x * 256 * kReorderPieces + threadIdx.x;
  const int64_t ph = blockIdx.y;  // plane * heads + head
  const int64_t plane = ph / a.heads, head = ph - plane * a.heads;
  const int64_t head_pieces = a.capacity * (kD / 8);
  const int64_t row_pieces = (int64_t)a.heads * head_pieces;
  u32x4* base = reinterpret_cast<u32x4*>(a.cache) + plane * a.rows * row_pieces +
                head * head_pieces;
  int par[kReorderMaxRows];
#pragma unroll
  for (int r = 0; r < kReorderMaxRows; ++r) {
    par[r] = r;
    if (r < a.rows) {
      const int64_t p = a.parents[r];
      if (p >= 0 && p < a.rows) par[r] = (int)p;
    }
  }
  // Every source piece of this thread is read before any is written, so
  // rows that exchange caches need no staging copy.
  u32x4 v[kReorderMaxRows][kReorderPieces];
#pragma unroll
  for (int r = 0; r < kReorderMaxRows; ++r) {
    if (par[r] == r) continue;
#pragma unroll
    for (int i = 0; i < kReorderPieces; ++i) {
      const int64_t e = e0 + i * 256;
      if (e < pieces) v[r][i] = base[par[r] * row_pieces + e];
    }
  }
#pragma unroll
  for (int r = 0; r < kReorderMaxRows; ++r) {
    if (par[r] == r) continue;
#pragma unroll
    for (int i = 0; i < kReorderPieces; ++i) {
      const int64_t e = e0 + i * 256;
      if (e < pieces) base[r * row_pieces + e] = v[r][i];
    }
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

hipError_t launch_cache_reorder(const ReorderArgs& a, int64_t planes, hipStream_t stream) {
  const int64_t pieces = a.length * (kD / 8);
  const int64_t per_block = 256 * kReorderPieces;
  const dim3 grid((unsigned)((pieces + per_block - 1) / per_block), (unsigned)(planes * a.heads));
  hipLaunchKernelGGL(cache_reorder_kernel, grid, dim3(256), 0, stream, a);
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
