// Host-side launch interface between the C ABI (svq_api.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace svq {

// Output element types of the dequantize kernels: the C ABI's SVQ_F16,
// SVQ_F32 and SVQ_BF16 codes.
enum OutType { kOutF16 = 0, kOutF32 = 1, kOutBF16 = 2 };

struct GemvArgs {
  const uint16_t* x;     // fp16 [m, k]
  const uint8_t* q;      // SoA payload
  const uint16_t* s;     // fp16 scale bits
  const uint16_t* bias;  // fp16 [n] or nullptr
  void* y;               // [m, n] fp16 or fp32
  int n, k;
  int lg_g;         // log2 of the lanes that share a row
  int chunk_units;  // units of x staged in LDS at a time (chunked kernel)
  int y_f32;
  int waves;        // streaming waves in the grid (streaming kernel)
  int slots;        // row tiles per workgroup (MFMA kernel)
  int ksplit;       // K splits per row tile (MFMA kernel)
  // Fusions (streaming kernels only for the LayerNorm; fp16 y only):
  const uint16_t* ln_w;      // LayerNorm of every x row before the product:
  const uint16_t* ln_b;      //   fp16 [k] weight and bias (either may be nullptr)
  float ln_eps;              //   (no LayerNorm when both are nullptr)
  const uint16_t* residual;  // fp16 [m, n] added to the rounded output, or nullptr
  int act;                   // 0 none, 1 tanh-approximated GELU of the rounded output
  // K split across workgroups (streaming MFMA kernel): with `partial` set,
  // workgroup b takes K slice b % slices of every row and writes its raw sums
  // to partial[slice][m][n]; split_finish adds the slices and stores y.
  int slices;  // 2..kSplitMaxSlices with `partial`
  float* partial;
  // Work plan of the streaming MFMA kernel, filled on the host by
  // launch_gemv_mfma4 so that the kernel divides nothing: the grid is
  // (K slices) x (workgroups per K slice).
  int units;        // units of x per K slice (the whole row without slices)
  int tiles;        // row tiles of 4 rows (8 with two row sets per lane)
  int tile_groups;  // groups of 4 / ksplit consecutive tiles
  int wave_major;   // at most one tile per wave, in wave-major order
  int tiles_hi;     // tile groups of a workgroup below tiles_full; one fewer from there
  int tiles_full;
  int steps;        // ring steps per tile, all K ranges together
  int lg_ksplit;    // log2 of ksplit (1, 2 or 4)
  int short_prologue;  // Q5_0 three-block lanes: one ring step before x is staged
  // Per-wave phase stamps of the streaming MFMA kernel, written only by
  // libsvq_timeline.so (built with SVQ_TIMELINE); null otherwise.
  unsigned long long* stamps;
};

// Timeline builds: stamp slots per wave, [linear workgroup * 4 + wave][12]:
// 0 entry, 1 x staged, 2 first step done, 3 first tile summed, 4 end,
// 5 tiles of the wave, 6 x loads issued, 7 work split known; with a
// LayerNorm staged from registers 8 mean known, 9 variance known, 10
// normalized x in LDS; 11 unused.
constexpr int kTimelineSlots = 12;
constexpr int kSplitMaxSlices = 8;

struct GemvShape {
  int m;
  int rows_per_group;  // R: rows owned by one lane group
  int groups;          // workgroups in the grid
  int chunk_units;
  int lg_g;
};

// Kernel launchers (svq_gemv.hip, svq_dequant.hip).
hipError_t launch_gemv(const GemvArgs& a, const GemvShape& sh, int qtype,
                       hipStream_t stream);
int lds_bytes_per_unit(int qtype);
int units_per_block(int qtype);

// Streaming kernel (svq_gemv_stream.hip): waves per workgroup, LDS bytes it
// needs for x and the offset sums, its function pointer (for occupancy
// queries) and launcher.
constexpr int kStreamWavesPerGroup = 4;
// Extra LDS of the streaming kernels for the LayerNorm weight and bias.
inline size_t layer_norm_lds_bytes(int k, bool ln) {
  return ln ? (size_t)2 * ((k / 8 + 63) / 64 * 64) * 16 : 0;
}
size_t stream_lds_bytes(int qtype, int m, int k);
const void* stream_kernel(int qtype, int m, int rows, int wpg, bool ln = false);
hipError_t launch_gemv_stream(const GemvArgs& a, int qtype, int m, int rows, int wpg,
                              int groups, hipStream_t stream);

// MFMA kernel (svq_gemv_mfma.hip): blocks per step, LDS bytes, function
// pointer (for occupancy queries) and launcher.
int mfma_blocks_per_step(int qtype);
size_t mfma_lds_bytes(int qtype, int m, int k, int rows, int wpg, int ksplit);
const void* mfma_kernel(int qtype, int m, int rows);
hipError_t launch_gemv_mfma(const GemvArgs& a, int qtype, int m, int rows, int groups,
                            hipStream_t stream);

// Streaming MFMA kernel (svq_gemv_mfma4.hip), 1 <= M <= 8: function pointer
// and launcher (LDS layout and size as the vector streaming kernel).
const void* mfma4_kernel(int qtype, int m, int rows, bool ln = false);
size_t mfma4_lds_bytes(int qtype, int m, int k, int rows, int ksplit);
hipError_t launch_gemv_mfma4(const GemvArgs& a, int qtype, int m, int rows, int groups,
                             hipStream_t stream);

// Decode attention (svq_attention.hip): one new token per row against a
// [rows, kv_heads, capacity, 128] fp16 key/value cache.
struct AttnArgs {
  const uint16_t* qkv;     // fp16 [rows, qkv_stride]: q (heads x 128), k, v (kv_heads x 128 each)
  int64_t qkv_stride;      // elements between rows of qkv
  const uint16_t* cos;     // fp16 [128] rotary tables, or nullptr (no rotation)
  const uint16_t* sin;
  uint16_t* keys;          // fp16 cache of this layer
  uint16_t* values;
  int64_t capacity;        // slots per (row, kv head) in the cache
  const int64_t* position; // device scalar: the slot of the new token
  const uint16_t* bias;    // fp16 [span] additive score bias, or nullptr
  int window;              // > 0: slots j > position or j <= position - window masked
  int span;                // slots attended
  uint16_t* out;           // fp16 [rows, heads x 128]
  int kv_heads;
  float scale;             // score scale (head_dim^-0.5)
  float2* ml;              // workspace: (max score, sum of exponentials) per head and chunk
  float* acc;              // workspace: weighted sum of V [128] per head and chunk
  int nchunks;
};
// Merge of the chunk partials (second kernel of the attention).
struct AttnMerge {
  const float2* ml;
  const float* acc;
  uint16_t* out;
  int nchunks;
};
int attention_chunks(int span);
int64_t attention_ml_bytes(int rows, int heads, int span);
hipError_t launch_chunks(const AttnArgs& a, int rows, int group, hipStream_t stream);
int64_t attention_workspace_bytes(int rows, int heads, int kv_heads, int span);
hipError_t launch_decode_attention(const AttnArgs& a, int rows, int group, hipStream_t stream);
// Beam reorder of a [planes, rows, heads, capacity, 128] fp16 cache.
struct ReorderArgs {
  uint16_t* cache;
  int64_t capacity;          // slots per (plane, row, head)
  int64_t length;            // leading slots moved
  const int64_t* parents;    // device int64 [rows]
  int rows;
  int heads;
};
hipError_t launch_cache_reorder(const ReorderArgs& a, int64_t planes, hipStream_t stream);

// Survivor selection of a beam-sampling step (svq_beam_select).
constexpr int kBeamMaxRows = 8;
constexpr int kBeamMaxCandidates = 1024;  // beams x candidates per beam
struct BeamSelectArgs {
  const float* probs;         // [beams * vocab]
  const float* noise;         // [beams * vocab] Exp(1) draws
  const float* scores;        // [beams * vocab]
  const int64_t* candidates;  // [beams, ncand] token ids
  const uint8_t* seen_in;     // [beams, seen_pitch]
  uint8_t* seen_out;          // [beams, seen_pitch]
  int64_t seen_pitch;         // bytes per seen row, a multiple of 16
  float* running;             // [beams] out
  int64_t* parents;           // [beams] out
  int64_t* tokens;            // [beams] out
  int64_t* tokens_copy;       // [beams] out, or NULL
  int64_t vocab;
  int beams;
  int ncand;
  int draws;
  int compact;                // probs / scores are [beams, ncand] (per candidate)
};
hipError_t launch_beam_select(const BeamSelectArgs& a, hipStream_t stream);

// Candidate tokens of a beam-sampling step (svq_beam_candidates).
constexpr int kCandMaxVocab = 65536;
constexpr int kCandMax = 64;  // candidates per row
struct BeamCandArgs {
  const uint16_t* logits;  // fp16 [beams, vocab]
  const uint8_t* seen;     // [beams, seen_pitch]
  int64_t seen_pitch;
  const float* running;    // [beams]
  int64_t* candidates;     // [beams, kc] out
  float* scores;           // [beams, kc] out
  float* probs;            // [beams * kc] out
  int64_t* status;         // [2 + beams] out: draws possible, any overflow, overflow per row
  int vocab;
  int beams;
  int k;
  int kc;
  int keep;
  float penalty;
  float temperature;
  float top_p_cut;         // 1 - top_p
  int use_top_p;
  void* workspace;         // beam_candidates_workspace bytes, 8-byte aligned
};
int64_t beam_candidates_workspace(int beams, int vocab, int kc);
hipError_t launch_beam_candidates(const BeamCandArgs& a, hipStream_t stream);

hipError_t launch_dequant(const uint8_t* q, const uint16_t* s, void* out,
                          int64_t nblocks, int qtype, int out_dtype,
                          hipStream_t stream);
hipError_t launch_dequant_rows(const uint8_t* q, const uint16_t* s,
                               const int64_t* ids, int64_t nids, int64_t nrows,
                               int k, void* out, int qtype, int out_dtype,
                               hipStream_t stream);

}  // namespace svq
