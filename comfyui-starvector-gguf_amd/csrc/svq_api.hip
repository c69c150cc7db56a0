// C ABI of libsvq.so (declared in include/svq.h): argument validation, launch
// shape selection and error reporting. Every argument check runs before any
// HIP call, so rejected calls need no GPU.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>

#include "../../include/svq.h"
#include "svq_launch.h"

#if SVQ_TIMELINE
namespace svq {
hipError_t launch_timeline_read(const void* p, uint32_t bytes, int groups, uint32_t* sink,
                                unsigned long long* stamps, hipStream_t stream);
}
#endif

namespace {

#if SVQ_TIMELINE
unsigned long long* g_stamps = nullptr;  // svq_timeline_stamps
#endif

thread_local char g_error[256] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof g_error, fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  snprintf(g_error, sizeof g_error, "%s: %s", what, hipGetErrorString(e));
  return (int)e;
}

bool valid_qtype(int qtype) {
  return qtype == SVQ_Q4_0 || qtype == SVQ_Q5_0 || qtype == SVQ_Q8_0;
}

int payload_bytes(int qtype) {
  return qtype == SVQ_Q4_0 ? 16 : qtype == SVQ_Q5_0 ? 20 : 32;
}

bool aligned(const void* p, uintptr_t a) {
  return ((uintptr_t)p & (a - 1)) == 0;
}

static_assert(SVQ_F16 == svq::kOutF16 && SVQ_F32 == svq::kOutF32 && SVQ_BF16 == svq::kOutBF16,
              "the dequantize kernels take the ABI's element type codes");

// Whether the byte ranges [a, a + na) and [b, b + nb) share a byte (an
// absent array, NULL, overlaps nothing).
bool overlaps(const void* a, uint64_t na, const void* b, uint64_t nb) {
  if (!a || !b || !na || !nb) return false;
  const uintptr_t pa = (uintptr_t)a, pb = (uintptr_t)b;
  return pa < pb + nb && pb < pa + na;
}

// Launch-shape overrides for tuning sweeps and for tests that exercise every
// kernel: SVQ_PATH ("mfma4", "mfma", "stream" or "chunked"), SVQ_LG_G (log2 lanes per
// row, 0..6) and SVQ_ROWS (rows per lane group, 1 or 2) of the streaming and
// chunked kernels, SVQ_LDS_KB (LDS budget of the chunked kernel), and
// SVQ_MFMA_R (MFMA row tiles per wave, 1 or 2; for the streaming MFMA kernel
// 3 selects its three-units-per-lane Q5_0 variant), SVQ_MFMA_S (K splits, 1..16) and
// SVQ_MFMA_P (tile slots per workgroup) of the MFMA kernel, SVQ_GROUPS_PER_CU
// (1 or 2: the most workgroups per CU of the streaming MFMA kernel) and
// SVQ_GROUPS (its exact workgroup count). Read on every call, so a process may
// change them.
struct Tuning {
  int lg_g = -1;
  int rows = 0;
  int path = 0;  // 0 automatic, 1 streaming, 2 chunked, 3 mfma, 4 streaming mfma
  int lds_kb = 40;
  int mfma_r = 0, mfma_s = 0, mfma_p = 0;
  int groups_per_cu = 0;  // streaming MFMA kernel: workgroups per CU (1 or 2), 0 automatic
  int groups = 0;         // streaming MFMA kernel: workgroup count, 0 automatic
};

Tuning tuning() {
  Tuning t;
  if (const char* v = getenv("SVQ_LG_G")) t.lg_g = atoi(v);
  if (const char* v = getenv("SVQ_ROWS")) t.rows = atoi(v);
  if (const char* v = getenv("SVQ_PATH"))
    t.path = strcmp(v, "stream") == 0    ? 1
             : strcmp(v, "chunked") == 0 ? 2
             : strcmp(v, "mfma") == 0    ? 3
             : strcmp(v, "mfma4") == 0   ? 4
                                         : 0;
  if (const char* v = getenv("SVQ_LDS_KB")) t.lds_kb = atoi(v);
  if (const char* v = getenv("SVQ_MFMA_R")) t.mfma_r = atoi(v);
  if (const char* v = getenv("SVQ_MFMA_S")) t.mfma_s = atoi(v);
  if (const char* v = getenv("SVQ_MFMA_P")) t.mfma_p = atoi(v);
  if (const char* v = getenv("SVQ_GROUPS_PER_CU")) t.groups_per_cu = atoi(v);
  if (const char* v = getenv("SVQ_GROUPS")) t.groups = atoi(v);
  if (t.lg_g > 6) t.lg_g = 6;
  if (t.rows != 0 && t.rows != 1 && t.rows != 2) t.rows = 0;
  if (t.lds_kb < 4 || t.lds_kb > 64) t.lds_kb = 40;
  if (t.mfma_r < 1 || t.mfma_r > 3) t.mfma_r = 0;
  if (t.mfma_s < 0 || t.mfma_s > 16) t.mfma_s = 0;
  if (t.mfma_p < 0 || t.mfma_p > 16) t.mfma_p = 0;
  if (t.groups_per_cu != 1 && t.groups_per_cu != 2) t.groups_per_cu = 0;
  if (t.groups < 0 || t.groups > (1 << 16)) t.groups = 0;
  return t;
}

// Lanes per row: as many as keep >= 8 units per lane, at most a wave.
int base_lg_g(int units) {
  int lg_g = 6;
  while (lg_g > 0 && (units >> lg_g) < 8) --lg_g;
  return lg_g;
}

svq::GemvShape choose_chunked_shape(int m, int n, int k, int qtype, const Tuning& tu) {
  svq::GemvShape sh;
  sh.m = m;
  const int units = (k / 32) * svq::units_per_block(qtype);
  const int lg_g = tu.lg_g >= 0 ? tu.lg_g : base_lg_g(units);
  sh.lg_g = lg_g;
  const int row_groups_per_wave = 64 >> lg_g;
  int rows = 1;
  if (m >= 2 && n / (row_groups_per_wave * 2 * 4) >= 512) rows = 2;
  if (tu.rows) rows = tu.rows;
  sh.rows_per_group = rows;
  const int rows_per_group = 4 * row_groups_per_wave * rows;
  sh.groups = (n + rows_per_group - 1) / rows_per_group;
  int chunk = (tu.lds_kb * 1024) / (m * svq::lds_bytes_per_unit(qtype));
  if (chunk > units) chunk = units;
  if (chunk < 1) chunk = 1;
  sh.chunk_units = chunk;
  return sh;
}

// Compute units of the current device and resident waves per CU of a
// streaming kernel with a given LDS size, cached (host queries only).
std::mutex g_cache_mu;
std::map<int, int> g_cus;
std::map<std::tuple<int, const void*, int, size_t>, int> g_waves_per_cu;

int device_cus(int dev) {
  std::lock_guard<std::mutex> lock(g_cache_mu);
  auto it = g_cus.find(dev);
  if (it != g_cus.end()) return it->second;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  g_cus[dev] = cus;
  return cus;
}

int waves_per_cu(int dev, const void* fn, int wpg, size_t lds) {
  std::lock_guard<std::mutex> lock(g_cache_mu);
  const auto key = std::make_tuple(dev, fn, wpg, lds);
  auto it = g_waves_per_cu.find(key);
  if (it != g_waves_per_cu.end()) return it->second;
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, wpg * 64, lds) != hipSuccess ||
      blocks <= 0)
    blocks = 1;
  g_waves_per_cu[key] = blocks * wpg;
  return blocks * wpg;
}

constexpr size_t kStreamLdsMax = 156 * 1024;  // nearly all of a CU's 160 KB
// Persistent launches with more tiles than this many workgroups per CU use
// exactly this many per CU.
constexpr int kPersistentGroupsPerCu = 2;

// Workgroups of a persistent launch that needs `want` of them (one tile
// group each): a whole number of workgroups per CU, at most
// kPersistentGroupsPerCu, so that wave-major tile numbering loads every CU
// alike; never more than the `cap` the GPU keeps resident.
int balanced_groups(int want, int cus, int cap) {
  const int per_cu = std::min((want + cus - 1) / cus, kPersistentGroupsPerCu);
  const int groups = per_cu * cus;
  return groups <= cap ? groups : std::min(want, cap);
}

// Streaming launch: lanes per row and rows per lane group chosen so that the
// row tiles cover every resident wave (largest tiles first, which reuse x
// the most); when there are more tiles than resident waves, the wave count is
// trimmed so that every wave gets the same number of tiles, as long as that
// keeps every CU busy, and capped at two workgroups per CU. Returns false
// when x does not fit in LDS or a buffer
// exceeds the 2^31-byte ranges the kernel addresses.
bool choose_stream(int m, int n, int k, int qtype, const Tuning& tu, int* lg_out,
                   int* rows_out, int* wpg_out, int* waves_out, int* groups_out,
                   int* wmax_out = nullptr, size_t extra_lds = 0) {
  if (tu.path == 2) return false;
  const size_t lds = svq::stream_lds_bytes(qtype, m, k) + extra_lds;
  const uint64_t q_bytes = (uint64_t)n * (k / 32) * payload_bytes(qtype);
  if (lds > kStreamLdsMax || q_bytes >= (1ull << 31) || (uint64_t)n * (k / 16) >= (1ull << 31))
    return false;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  const int cus = device_cus(dev);
  const int wpg = svq::kStreamWavesPerGroup;
  const int units = (k / 32) * svq::units_per_block(qtype);
  const int lg0 = base_lg_g(units);
  // Widening a row group below 4 units per lane costs more in per-wave
  // overhead (staging, reduction, idle lanes) than the extra waves recover.
  int lg_cap = lg0;
  while (lg_cap < 6 && (units >> (lg_cap + 1)) >= 4) ++lg_cap;
  int lg = lg0, rows = 2, wmax = 0, tiles = 0;
  for (;;) {
    wmax = cus * waves_per_cu(dev, svq::stream_kernel(qtype, m, rows, wpg, extra_lds > 0), wpg, lds);
    tiles = (n + ((64 >> lg) * rows) - 1) / ((64 >> lg) * rows);
    if (tiles >= wmax) break;
    if (rows == 2) rows = 1;
    else if (lg < lg_cap) ++lg;
    else break;
  }
  if (tu.lg_g >= 0) lg = tu.lg_g;
  if (tu.rows) rows = tu.rows;
  if (tu.lg_g >= 0 || tu.rows) {
    wmax = cus * waves_per_cu(dev, svq::stream_kernel(qtype, m, rows, wpg, extra_lds > 0), wpg, lds);
    tiles = (n + ((64 >> lg) * rows) - 1) / ((64 >> lg) * rows);
  }
  int waves = tiles < wmax ? tiles : wmax;
  const int rounds = (tiles + waves - 1) / waves;
  const int balanced = (tiles + rounds - 1) / rounds;
  if (balanced >= wmax - wmax / 16) waves = balanced;
  // Two workgroups per CU at most, as the streaming MFMA launch.
  const int wcap = kPersistentGroupsPerCu * wpg * cus;
  if (tiles > wcap && wcap <= wmax) waves = wcap;
  *lg_out = lg;
  *rows_out = rows;
  *wpg_out = wpg;
  *waves_out = waves;
  *groups_out = balanced_groups((waves + wpg - 1) / wpg, cus, wmax / wpg);
  if (wmax_out) *wmax_out = wmax;
  return true;
}

constexpr int kMfmaMinRows = 5;  // smallest M sent to the MFMA kernel by default

// Streaming MFMA launch (M <= 8): row tiles of 4 rows (8 with two row sets
// per lane) over 16 unit slots. Variant (the `rows` code): 3 = consecutive
// units per lane (three Q4_0 / Q5_0 blocks, needs units % 48 == 0; one Q8_0
// block), 2 = two row sets per lane, 1 = one. The 4 waves of a workgroup
// split K (S = 2 or 4) and add their partial sums through LDS: by default
// S = 2 when single-row-set tiles fill a quarter of the resident waves or
// fewer, and for long Q8_0 rows; otherwise as SVQ_MFMA_S asks. Workgroups
// are persistent over tile groups; without split K their count is a whole
// number per CU, at most two (balanced_groups).
bool choose_mfma4(int m, int n, int k, int qtype, const Tuning& tu, int* rows_out,
                  int* ksplit_out, int* groups_out, int* wmax_out, size_t extra_lds = 0) {
  if ((tu.path != 4 && tu.path != 0) || m > 8) return false;
  // M = 5..8 runs two A halves per unpacked weight operand. Measured at the
  // 8B shapes against the 16x16x32 kernel: faster for Q5_0 and Q8_0 at every
  // M (Q5_0 c_fc 39.1 -> 22.6 us, Q8_0 lm_head 94.8 -> 51.0 us at M = 5; at M
  // = 8 Q5_0 c_fc 31.0 -> 26.6 us, lm_head 52.1 -> 45.3 us, Q8_0 lm_head 75.8
  // -> 65.1 us) and for Q4_0 at every M (at M = 8: c_fc 24.5 -> 21.5 us,
  // lm_head 40.2 -> 36.8 us, qkv 13.0 -> 12.2 us, 2048 x 8192 13.4 -> 13.5
  // us with one row set).
  // Automatic choice (measured at the StarCoder2-8B and GPTBigCode-1B shapes):
  // the matrix-core path wins for Q5_0 at every M and for Q4_0 / Q8_0 from
  // M = 2; at M = 1 the vector path's dot products are cheap enough, except
  // on matrices of 32 MiB or less with K = 4608 (4608 x 4608 and 5632 x
  // 4608), or up to K = 8192 for Q8_0 (8192 x 2048).
  const uint64_t q_bytes = (uint64_t)n * (k / 32) * payload_bytes(qtype);
  if (tu.path == 0 && qtype != SVQ_Q5_0 && m < 2) {
    const bool k_ok = qtype == SVQ_Q8_0 ? k <= 8192 : (k >= 4096 && k <= 6144);
    if (q_bytes > (32u << 20) || !k_ok) return false;
  }
  if (q_bytes >= (1ull << 31) || (uint64_t)n * (k / 16) >= (1ull << 31)) return false;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  const int cus = device_cus(dev);
  const int wpg = svq::kStreamWavesPerGroup;
  const int units = (k / 32) * svq::units_per_block(qtype);
  // Variant 3 reads consecutive units per lane: three blocks (Q4_0 / Q5_0,
  // whole steps only: units % 48 == 0) or one Q8_0 block (two units).
  const bool multi = qtype == SVQ_Q8_0 || units % 48 == 0;
  const int unit_run = qtype == SVQ_Q8_0 ? 2 : 3;
  // Defaults: variant 3 for Q5_0 and Q8_0 (measured 2-9% faster than two row
  // sets at K = 4608 and 18432). Q4_0 takes it at M = 2..4 for matrices up
  // to 64 MiB (8B beam-2 decode 468 -> 479 steps/s; qkv 5632 x 4608 at M = 2
  // 7.7 against 8.1 us; at M = 3..4 c_fc 16.1 -> 14.6 us and c_proj's slices
  // 18.1 -> 16.9 us). Larger Q4_0 matrices read one unit per lane in two row
  // sets, whose loads cover whole cache lines with the non-temporal hint
  // (lm_head 49152 x 4608 at M = 2: 26.6 -> 24.0 us back to back, 27.2 ->
  // 26.3 us inside the decode step). In back-to-back launches one-unit lanes
  // also win on c_fc and c_proj's slices at M = 2 (13.5 -> 13.0 and 16.1 ->
  // 15.4 us), but inside the decode step, behind the kernels that write
  // their x, they lose (15.1 -> 16.6 and 13.1 -> 13.8 us). M = 1 keeps two
  // row sets, which share each x read. With two A halves (M >= 5) two row
  // sets win for Q5_0 (c_fc 24.2 -> 22.6 us, lm_head 46.5 -> 40.2 us at M =
  // 5) and for Q8_0 at M = 8 (lm_head 85.5 -> 65.1 us); Q8_0 keeps
  // whole-block lanes at M = 5..7.
  const bool q4_rows3 = m >= 2 && m <= 4 && q_bytes <= (64ull << 20);
  // Q8_0 rows of 2048 weights or fewer at M <= 2 take two row sets of
  // one-unit lanes, whose loads cover whole cache lines (non-temporal), on
  // matrices of more than 4096 rows: 8192 x 2048 at M = 1 7.0 -> 6.3 us, M =
  // 2 7.1 -> 6.6 us; 49152 x 2048 at M = 2 21.2 -> 20.5 us. Fewer rows keep
  // whole-block lanes (2304 x 2048 at M = 2: 4.6 against 5.9 us). At K =
  // 4608 whole-block lanes stay faster, except on matrices over 128 MiB at M
  // = 2..4, where enough row tiles remain to balance two row sets (lm_head
  // 49152 x 4608: 45.1 -> 42.1 us at M = 2, 47.5 -> 43.9 us at M = 4).
  const bool q8_short = qtype == SVQ_Q8_0 && m <= 2 && k <= 2048 && n > 4096;
  const bool q8_large = qtype == SVQ_Q8_0 && m >= 2 && m <= 4 && q_bytes > (128ull << 20);
  const bool rows3 = q8_short || q8_large ? false
                     : m <= 4 ? qtype != SVQ_Q4_0 || q4_rows3
                              : qtype == SVQ_Q8_0 && m < 8;
  int rows = tu.mfma_r ? tu.mfma_r : (rows3 && multi ? 3 : 2);
  if (rows == 3 && !multi) rows = 2;
  int wmax = 0, tiles = 0;
  size_t lds = 0;
  for (;;) {
    // Occupancy of the launch without split K (no LDS for partial sums): at
    // M = 8 (Q5_0, K = 4608) those 2 KB decide between one and two workgroups
    // per CU (c_fc 31.2 -> 26.6 us).
    lds = svq::mfma4_lds_bytes(qtype, m, k, rows, 1) + extra_lds;
    if (lds > kStreamLdsMax) return false;
    wmax = cus * waves_per_cu(dev, svq::mfma4_kernel(qtype, m, rows, extra_lds > 0), wpg, lds);
    const int tile_rows = rows == 2 ? 8 : 4;
    tiles = (n + tile_rows - 1) / tile_rows;
    // Two row sets per lane share each x read; measured faster down to an
    // eighth of the resident waves (Q4_0 / Q8_0 at K = 4608, M = 2..4), and
    // for Q4_0 at M = 7..8 above a quarter (at M = 8: 2048 x 8192, a quarter
    // exactly, one row set 13.6 against 15.5 us; 2304 x 2048 6.9 against 7.9
    // us; 4608 x 4608 two row sets 12.1 against 13.9 us; at M = 5 the
    // quarter rule put 4608 x 4608 on one row set, 11.4 against 10.8 us).
    const bool keep_two = qtype == SVQ_Q4_0 && m >= 7 ? 4 * (int64_t)tiles > wmax
                                                       : 8 * (int64_t)tiles >= wmax;
    if (tiles >= wmax || rows != 2 || tu.mfma_r || keep_two) break;
    rows = 1;
  }
  // Long rows with too few tiles to fill the GPU go to the vector kernel,
  // which spreads a row over 64 lanes: measured faster than splitting K here,
  // except for Q8_0 whole-block lanes split in two (4608 x 18432, M = 2:
  // 24.8 us against 27.8 us).
  const bool long_q8 = qtype == SVQ_Q8_0 && rows == 3 && k > 8192;
  if (tu.path == 0 && k > 8192 && tiles < wmax && !long_q8) return false;
  const int per_step = 16 * (rows == 3 ? unit_run : 1);
  const int steps = (units + per_step - 1) / per_step;
  int ksplit = 1;
  if (tu.mfma_s == 2 || tu.mfma_s == 4) {
    ksplit = tu.mfma_s;
  } else if (tu.mfma_s == 0 && rows == 1 && 4 * (int64_t)tiles <= wmax && steps >= 8) {
    ksplit = 2;  // a quarter of the waves or fewer: halve K per wave
  } else if (tu.mfma_s == 0 && long_q8) {
    ksplit = 2;
  }
  if (ksplit > steps) ksplit = 1;  // every wave needs at least one step
  if (ksplit > 1) {  // the partial sums' LDS: occupancy again, or no split
    const size_t lds_split = svq::mfma4_lds_bytes(qtype, m, k, rows, ksplit) + extra_lds;
    if (lds_split > kStreamLdsMax)
      ksplit = 1;
    else
      wmax = cus * waves_per_cu(dev, svq::mfma4_kernel(qtype, m, rows, extra_lds > 0), wpg,
                                lds_split);
  }
  const int slots = wpg / ksplit;
  const int tile_groups = (tiles + slots - 1) / slots;
  int cap = wmax / wpg;
  if (tu.groups_per_cu && cap > tu.groups_per_cu * cus) cap = tu.groups_per_cu * cus;
  int groups = tile_groups < cap ? tile_groups : cap;
  const int rounds = (tile_groups + groups - 1) / groups;
  groups = (tile_groups + rounds - 1) / rounds;
  // Without split K (wave-major tiles, one tile or none per wave when the
  // matrix is short) the workgroup count is a whole number of workgroups per
  // CU, at most two, so that every CU holds as many tiles as the next: two
  // per CU streams faster than filling every resident slot (measured 5-18%
  // on the 8B c_fc and lm_head shapes at M = 1..4), and rounding short
  // matrices up to whole CUs 3-12% on qkv and o_proj.
  if (ksplit == 1) groups = balanced_groups(tile_groups, cus, cap);
  if (tu.groups) groups = std::min(tu.groups, std::min(tile_groups, cap));
  *rows_out = rows;
  *ksplit_out = ksplit;
  *groups_out = groups;
  *wmax_out = wmax;
  return true;
}

// MFMA launch: 16-row tiles, split along K until tiles x splits give about
// 16 waves per CU (each split keeping >= 2 steps), persistent workgroups
// trimmed so that each processes the same number of tile groups. Returns false
// when the shape or alignment does not suit the kernel: K must be a whole
// number of steps (4 blocks, 2 for Q8_0), the scales 4-byte aligned, x and
// its offset sums must fit in LDS, and the arrays below 2^31 bytes.
bool choose_mfma(int m, int n, int k, int qtype, const Tuning& tu, const void* s, int* rows_out,
                 int* slots_out, int* ksplit_out, int* groups_out) {
  if (tu.path == 1 || tu.path == 2 || tu.path == 4) return false;
  // Automatic choice: the matrix cores pay off once the per-weight dot work
  // (M fp32 FMAs per weight on the vector path) outweighs the MFMA path's
  // fixed cost; measured crossover at MI355X decoder shapes is M = 4..5.
  if (tu.path == 0 && m < kMfmaMinRows) return false;
  const int kb = k / 32;
  const int bps = svq::mfma_blocks_per_step(qtype);
  if (kb % bps || !aligned(s, 4)) return false;
  const int steps = kb / bps;
  const uint64_t q_bytes = (uint64_t)n * kb * payload_bytes(qtype);
  if (q_bytes >= (1ull << 31) || (uint64_t)n * kb * 2 >= (1ull << 31)) return false;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  const int cus = device_cus(dev);
  const int rows = tu.mfma_r == 1 || tu.mfma_r == 2 ? tu.mfma_r : (m >= kMfmaMinRows ? 2 : 1);
  const int tiles = (n + 16 * rows - 1) / (16 * rows);
  int ksplit = 1;
  if (tu.mfma_s) {
    ksplit = tu.mfma_s;
  } else {
    while (ksplit < 16 && (int64_t)tiles * 2 * ksplit <= (int64_t)cus * 16 &&
           steps >= 4 * ksplit)
      ksplit *= 2;
  }
  if (ksplit > steps) ksplit = steps;  // every wave needs at least one step
  int slots = tu.mfma_p ? tu.mfma_p : (ksplit >= 4 ? 1 : 4 / ksplit);
  if (slots * ksplit > 16) slots = 16 / ksplit;
  if (slots < 1) return false;
  const int wpg = slots * ksplit;
  const size_t lds = svq::mfma_lds_bytes(qtype, m, k, rows, wpg, ksplit);
  if (lds > kStreamLdsMax) return false;
  const int per_cu = waves_per_cu(dev, svq::mfma_kernel(qtype, m, rows), wpg, lds) / wpg;
  const int tile_groups = (tiles + slots - 1) / slots;
  int groups = tile_groups < cus * per_cu ? tile_groups : cus * per_cu;
  const int rounds = (tile_groups + groups - 1) / groups;
  groups = (tile_groups + rounds - 1) / rounds;
  *rows_out = rows;
  *slots_out = slots;
  *ksplit_out = ksplit;
  *groups_out = groups;
  return true;
}

// Fused prologue / epilogue of svq_gemv_fused (all null / zero for svq_gemv).
struct Fusion {
  const uint16_t* ln_w = nullptr;
  const uint16_t* ln_b = nullptr;
  float ln_eps = 0.f;
  const uint16_t* residual = nullptr;
  int act = SVQ_ACT_NONE;
  bool layer_norm() const { return ln_w || ln_b; }
};

// K split across workgroups, for a caller that provides a workspace: rows
// longer than 8192 weights at M = 2..8 without a LayerNorm are cut into SL
// slices of at most 4608 weights (SL divides K / 32). Each workgroup stages
// only its slice of x (18 KB at M = 2 instead of the whole row's 74 KB) and
// writes raw partial sums; a second kernel adds the slices in order and
// stores y. Measured on 4608 x 18432: M = 2 2.2-3.0 us faster (Q4_0 /
// Q5_0), M = 4 7.5 us; at M = 1 the vector kernel's single pass is faster.
// At M = 5..8 x of a long row does not fit in LDS at all (the chunked kernel,
// 47-94 us on 4608 x 18432), so every slice runs the streaming MFMA kernel.
// Returns SL, or 0 when the shape stays one pass.
int split_slices(int m, int k, bool layer_norm) {
  if (layer_norm || m < 2 || m > 8 || k <= 8192) return 0;
  const int kb = k / 32;
  for (int sl = 2; sl <= svq::kSplitMaxSlices; ++sl)
    if (kb % sl == 0 && k / sl <= 4608) return sl;
  return 0;
}

int64_t split_workspace_bytes(int m, int n, int k) {
  const int sl = split_slices(m, k, false);
  return sl ? (int64_t)sl * m * n * 4 : 0;
}

// Scratch of svq_gemv_split_static: the K split's fp32 partial sums in a
// file-scope device array instead of a caller's workspace. Every GPU the
// library runs on holds its own copy at its own address until the process
// ends. In host code `scratch` names a host-side stand-in, never the device
// memory: its device address is resolved once per device
// (hipGetSymbolAddress, with that device current) and only that address is
// passed to kernels. The partial sums are written in full before they are
// read within one call, so nothing needs clearing between calls.
constexpr int64_t kStaticScratchBytes = SVQ_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];
std::map<int, void*> g_scratch;  // device -> device address of `scratch`

// The current device's address of `scratch` (0, or a positive hipError_t).
int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_cache_mu);
  auto it = g_scratch.find(dev);
  if (it == g_scratch.end()) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress of the static scratch");
    if (!ptr) return hip_fail(hipErrorInvalidSymbol, "static scratch has no device address");
    it = g_scratch.emplace(dev, ptr).first;
  }
  *out = it->second;
  return 0;
}

// Every argument check of a GEMV call, before any HIP call (0 or an SVQ_E*
// code with the message set).
int check_gemv(const void* x, const uint8_t* q, const uint16_t* s, const uint16_t* bias,
               void* y, int m, int n, int k, int qtype, int y_dtype, const Fusion& f,
               void* workspace, int64_t workspace_bytes) {
  if (!valid_qtype(qtype)) return fail(SVQ_E_QTYPE, "unsupported qtype %d", qtype);
  if (m < 1 || m > SVQ_MAX_ROWS)
    return fail(SVQ_E_SHAPE, "m=%d outside 1..%d", m, SVQ_MAX_ROWS);
  if (n < 1 || k < 32 || k % 32)
    return fail(SVQ_E_SHAPE, "invalid matrix dimensions n=%d k=%d", n, k);
  if (k > (1 << 24) || n > (1 << 30))
    return fail(SVQ_E_RANGE, "n=%d k=%d exceeds the supported range", n, k);
  if (!x || !q || !s || !y) return fail(SVQ_E_NULL, "NULL x, q, s or y");
  if (y_dtype != SVQ_F16 && y_dtype != SVQ_F32)
    return fail(SVQ_E_DTYPE, "y_is_fp32 %d is not 0 (fp16) or 1 (fp32)", y_dtype);
  if (!aligned(x, 16) || !aligned(q, qtype == SVQ_Q5_0 ? 4 : 16) ||
      !aligned(s, 2) || (bias && !aligned(bias, 2)) ||
      !aligned(y, y_dtype == SVQ_F32 ? 4 : 2))
    return fail(SVQ_E_ALIGN, "misaligned pointer (x and q need 16 bytes)");
  // Per-wave 32-bit offsets: up to 128 rows of payload stay below 2^31 bytes,
  // the offset the kernels use for loads that must not touch memory.
  if ((uint64_t)(k / 32) * payload_bytes(qtype) * 128 >= (1ull << 31))
    return fail(SVQ_E_RANGE, "row of %d weights too long", k);
  // y is written while other workgroups still read the inputs (each stages
  // all of x, the LayerNorm parameters, its weight rows, bias and residual),
  // so y may share no byte with any of them; the residual may be y itself
  // (each element is read, then written, by one thread). The workspace is
  // written too.
  {
    const uint64_t y_bytes = (uint64_t)m * n * (y_dtype == SVQ_F32 ? 4 : 2);
    const uint64_t blocks = (uint64_t)n * (k / 32);
    const struct {
      const void* p;
      uint64_t bytes;
    } inputs[] = {{x, (uint64_t)m * k * 2},
                  {q, blocks * payload_bytes(qtype)},
                  {s, blocks * 2},
                  {bias, (uint64_t)n * 2},
                  {f.ln_w, (uint64_t)k * 2},
                  {f.ln_b, (uint64_t)k * 2},
                  {f.residual != y ? f.residual : nullptr, (uint64_t)m * n * 2}};
    for (const auto& in : inputs)
      if (overlaps(y, y_bytes, in.p, in.bytes))
        return fail(SVQ_E_SHAPE, "y overlaps an input (x, weights, bias, LayerNorm or residual)");
    if (workspace && workspace_bytes > 0) {
      if (overlaps(workspace, (uint64_t)workspace_bytes, y, y_bytes) ||
          overlaps(workspace, (uint64_t)workspace_bytes, f.residual, (uint64_t)m * n * 2))
        return fail(SVQ_E_SHAPE, "workspace overlaps y or the residual");
      for (const auto& in : inputs)
        if (overlaps(workspace, (uint64_t)workspace_bytes, in.p, in.bytes))
          return fail(SVQ_E_SHAPE, "workspace overlaps an input");
    }
  }
  return 0;
}

int gemv_impl(const void* x, const uint8_t* q, const uint16_t* s, const uint16_t* bias,
              void* y, int m, int n, int k, int qtype, int y_dtype, const Fusion& f,
              void* stream, void* workspace = nullptr, int64_t workspace_bytes = 0) {
  if (const int rc = check_gemv(x, q, s, bias, y, m, n, k, qtype, y_dtype, f, workspace,
                               workspace_bytes))
    return rc;
  const Tuning tu = tuning();
  svq::GemvArgs a{};
#if SVQ_TIMELINE
  a.stamps = g_stamps;
#endif
  a.x = static_cast<const uint16_t*>(x);
  a.q = q;
  a.s = s;
  a.bias = bias;
  a.y = y;
  a.n = n;
  a.k = k;
  a.y_f32 = y_dtype == SVQ_F32;
  a.ln_w = f.ln_w;
  a.ln_b = f.ln_b;
  a.ln_eps = f.ln_eps;
  a.residual = f.residual;
  a.act = f.act;
  int lg = 0, rows = 0, wpg = 0, waves = 0, groups = 0, slots = 0, ksplit = 0;
  hipError_t e;
  int wmax = 0;
  // The LayerNorm runs in the x staging of the two streaming kernels.
  const size_t ln_lds = svq::layer_norm_lds_bytes(k, f.layer_norm());
  // K split: each slice planned as a K / SL matrix of n * SL rows; the
  // workgroup count a multiple of SL (workgroup b takes slice b % SL).
  const int sl = workspace ? split_slices(m, k, f.layer_norm()) : 0;
  Tuning tu_split = tu;  // slices always on the streaming MFMA kernel
  if (tu_split.path == 0) tu_split.path = 4;
  if (sl && workspace_bytes >= split_workspace_bytes(m, n, k) &&
      choose_mfma4(m, n * sl, k / sl, qtype, tu_split, &rows, &ksplit, &groups, &wmax)) {
    a.ksplit = 1;
    a.slices = sl;
    a.partial = static_cast<float*>(workspace);
    groups = (groups + sl - 1) / sl * sl;
    e = svq::launch_gemv_mfma4(a, qtype, m, rows, groups, static_cast<hipStream_t>(stream));
  } else if (choose_mfma4(m, n, k, qtype, tu, &rows, &ksplit, &groups, &wmax, ln_lds)) {
    a.ksplit = ksplit;
    e = svq::launch_gemv_mfma4(a, qtype, m, rows, groups, static_cast<hipStream_t>(stream));
  } else if (!f.layer_norm() &&
             choose_mfma(m, n, k, qtype, tu, s, &rows, &slots, &ksplit, &groups)) {
    a.slots = slots;
    a.ksplit = ksplit;
    e = svq::launch_gemv_mfma(a, qtype, m, rows, groups, static_cast<hipStream_t>(stream));
  } else if (choose_stream(m, n, k, qtype, f.layer_norm() ? Tuning{} : tu, &lg, &rows, &wpg,
                           &waves, &groups, nullptr, ln_lds)) {
    a.lg_g = lg;
    a.waves = waves;
    e = svq::launch_gemv_stream(a, qtype, m, rows, wpg, groups,
                                static_cast<hipStream_t>(stream));
  } else if (!f.layer_norm()) {
    const svq::GemvShape sh = choose_chunked_shape(m, n, k, qtype, tu);
    a.lg_g = sh.lg_g;
    a.chunk_units = sh.chunk_units;
    e = svq::launch_gemv(a, sh, qtype, static_cast<hipStream_t>(stream));
  } else {
    return fail(SVQ_E_SHAPE, "LayerNorm fusion needs x (m=%d, k=%d) to fit in LDS", m, k);
  }
  if (e != hipSuccess) return hip_fail(e, "svq_gemv launch");
  return 0;
}

}  // namespace

namespace svq {
// Error reporting for the library's host-only sources (svq_gguf.cpp).
int set_error(int code, const char* msg) { return fail(code, "%s", msg); }
}  // namespace svq

extern "C" {

int svq_abi_version(void) { return SVQ_ABI_VERSION; }

#if SVQ_TIMELINE
void svq_timeline_stamps(void* stamps) { g_stamps = static_cast<unsigned long long*>(stamps); }

int svq_timeline_read(const void* p, uint64_t bytes, int groups, void* sink, void* stamps,
                      void* stream) {
  if (!p || !sink || !stamps || bytes % 1024 || bytes >= (1ull << 31) || groups < 1 ||
      groups > 4096)
    return fail(SVQ_E_SHAPE, "invalid timeline read");
  const hipError_t e =
      svq::launch_timeline_read(p, (uint32_t)bytes, groups, static_cast<uint32_t*>(sink),
                                static_cast<unsigned long long*>(stamps),
                                static_cast<hipStream_t>(stream));
  return e == hipSuccess ? 0 : hip_fail(e, "timeline read launch");
}
#endif

const char* svq_last_error(void) { return g_error; }

int svq_gemv(const void* x, const uint8_t* q, const uint16_t* s,
             const uint16_t* bias, void* y, int m, int n, int k, int qtype,
             int y_is_fp32, void* stream) {
  // y_is_fp32 is 0 (SVQ_F16) or 1 (SVQ_F32); anything else is rejected.
  return gemv_impl(x, q, s, bias, y, m, n, k, qtype, y_is_fp32, Fusion{}, stream);
}

int64_t svq_gemv_split_workspace(int m, int n, int k, int qtype) {
  if (!valid_qtype(qtype)) return fail(SVQ_E_QTYPE, "unsupported qtype %d", qtype);
  if (m < 1 || m > SVQ_MAX_ROWS || n < 1 || k < 32 || k % 32 || k > (1 << 24) || n > (1 << 30))
    return fail(SVQ_E_SHAPE, "invalid GEMV shape m=%d n=%d k=%d", m, n, k);
  return split_workspace_bytes(m, n, k);
}

int svq_gemv_split(const void* x, const uint8_t* q, const uint16_t* s, const uint16_t* bias,
                   void* y, int m, int n, int k, int qtype, const uint16_t* residual,
                   int activation, void* workspace, int64_t workspace_bytes, void* stream) {
  if (activation != SVQ_ACT_NONE && activation != SVQ_ACT_GELU_TANH)
    return fail(SVQ_E_DTYPE, "unsupported activation %d", activation);
  if ((residual && !aligned(residual, 2)) || (workspace && !aligned(workspace, 16)))
    return fail(SVQ_E_ALIGN, "misaligned residual or workspace");
  if (workspace_bytes < 0) return fail(SVQ_E_WORKSPACE, "negative workspace size");
  Fusion f;
  f.residual = residual;
  f.act = activation;
  return gemv_impl(x, q, s, bias, y, m, n, k, qtype, SVQ_F16, f, stream, workspace,
                   workspace_bytes);
}

int svq_gemv_split_static(const void* x, const uint8_t* q, const uint16_t* s,
                          const uint16_t* bias, void* y, int m, int n, int k, int qtype,
                          const uint16_t* residual, int activation, void* stream) {
  // The checks of svq_gemv_split first (no HIP call before them), then the
  // scratch: its size against the shape, its address on this device.
  if (activation != SVQ_ACT_NONE && activation != SVQ_ACT_GELU_TANH)
    return fail(SVQ_E_DTYPE, "unsupported activation %d", activation);
  if (residual && !aligned(residual, 2)) return fail(SVQ_E_ALIGN, "misaligned residual");
  Fusion f;
  f.residual = residual;
  f.act = activation;
  if (const int rc = check_gemv(x, q, s, bias, y, m, n, k, qtype, SVQ_F16, f, nullptr, 0))
    return rc;
  const int64_t need = split_workspace_bytes(m, n, k);
  if (need > kStaticScratchBytes)
    return fail(SVQ_E_WORKSPACE,
                "m=%d n=%d k=%d needs %lld bytes of split-K scratch; the static scratch holds "
                "%lld (use svq_gemv_split with a workspace)",
                m, n, k, (long long)need, (long long)kStaticScratchBytes);
  void* ptr = nullptr;
  if (need > 0)
    if (const int rc = scratch_address(&ptr)) return rc;
  return gemv_impl(x, q, s, bias, y, m, n, k, qtype, SVQ_F16, f, stream, ptr, need);
}

int svq_gemv_fused(const void* x, const uint8_t* q, const uint16_t* s, const uint16_t* bias,
                   void* y, int m, int n, int k, int qtype, const uint16_t* ln_weight,
                   const uint16_t* ln_bias, float ln_eps, const uint16_t* residual,
                   int activation, void* stream) {
  if (activation != SVQ_ACT_NONE && activation != SVQ_ACT_GELU_TANH)
    return fail(SVQ_E_DTYPE, "unsupported activation %d", activation);
  if ((ln_weight && !aligned(ln_weight, 16)) || (ln_bias && !aligned(ln_bias, 16)) ||
      (residual && !aligned(residual, 2)))
    return fail(SVQ_E_ALIGN, "misaligned LayerNorm parameters or residual");
  if ((ln_weight || ln_bias) && !(ln_eps >= 0.f))
    return fail(SVQ_E_SHAPE, "invalid LayerNorm eps");
  Fusion f;
  f.ln_w = ln_weight;
  f.ln_b = ln_bias;
  f.ln_eps = ln_eps;
  f.residual = residual;
  f.act = activation;
  return gemv_impl(x, q, s, bias, y, m, n, k, qtype, SVQ_F16, f, stream);
}

int svq_gemv_plan(int m, int n, int k, int qtype, int32_t* plan) {
  if (!valid_qtype(qtype)) return fail(SVQ_E_QTYPE, "unsupported qtype %d", qtype);
  if (m < 1 || m > SVQ_MAX_ROWS || n < 1 || k < 32 || k % 32)
    return fail(SVQ_E_SHAPE, "invalid shape m=%d n=%d k=%d", m, n, k);
  if (!plan) return fail(SVQ_E_NULL, "NULL plan");
  const Tuning tu = tuning();
  int lg = 0, rows = 0, wpg = 0, waves = 0, groups = 0, wmax = 0;
  for (int i = 0; i < 8; ++i) plan[i] = 0;
  int slots = 0, ksplit = 0;
  if (choose_mfma4(m, n, k, qtype, tu, &rows, &ksplit, &groups, &wmax)) {
    const int32_t p[8] = {4, ksplit, rows, svq::kStreamWavesPerGroup,
                          groups * svq::kStreamWavesPerGroup, groups, wmax, 0};
    for (int i = 0; i < 8; ++i) plan[i] = p[i];
  } else if (choose_mfma(m, n, k, qtype, tu, nullptr, &rows, &slots, &ksplit, &groups)) {
    const int32_t p[8] = {3, ksplit, rows, slots * ksplit, groups * slots * ksplit, groups, slots,
                          0};
    for (int i = 0; i < 8; ++i) plan[i] = p[i];
  } else if (choose_stream(m, n, k, qtype, tu, &lg, &rows, &wpg, &waves, &groups, &wmax)) {
    const int32_t p[8] = {1, lg, rows, wpg, waves, groups, wmax, 0};
    for (int i = 0; i < 8; ++i) plan[i] = p[i];
  } else {
    const svq::GemvShape sh = choose_chunked_shape(m, n, k, qtype, tu);
    const int32_t p[8] = {2, sh.lg_g, sh.rows_per_group, 4, sh.groups * 4, sh.groups, 0,
                          sh.chunk_units};
    for (int i = 0; i < 8; ++i) plan[i] = p[i];
  }
  return 0;
}

int svq_dequant(const uint8_t* q, const uint16_t* s, void* out,
                int64_t nblocks, int qtype, int out_dtype, void* stream) {
  if (!valid_qtype(qtype)) return fail(SVQ_E_QTYPE, "unsupported qtype %d", qtype);
  if (nblocks < 0) return fail(SVQ_E_SHAPE, "negative block count");
  if (out_dtype != SVQ_F32 && out_dtype != SVQ_F16 && out_dtype != SVQ_BF16)
    return fail(SVQ_E_DTYPE, "unsupported out_dtype %d", out_dtype);
  if (nblocks == 0) return 0;
  if (!q || !s || !out) return fail(SVQ_E_NULL, "NULL q, s or out");
  if (nblocks > (int64_t)1 << 36)
    return fail(SVQ_E_RANGE, "too many blocks (%lld)", (long long)nblocks);
  if (!aligned(q, qtype == SVQ_Q5_0 ? 4 : 16) || !aligned(s, 2) ||
      !aligned(out, 16))
    return fail(SVQ_E_ALIGN, "misaligned q or out (16 bytes required)");
  const hipError_t e = svq::launch_dequant(q, s, out, nblocks, qtype, out_dtype,
                                           static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "svq_dequant launch");
  return 0;
}

int svq_dequant_rows(const uint8_t* q, const uint16_t* s, const int64_t* ids,
                     int64_t nids, int64_t nrows, int k, void* out, int qtype,
                     int out_dtype, void* stream) {
  if (!valid_qtype(qtype)) return fail(SVQ_E_QTYPE, "unsupported qtype %d", qtype);
  if (nids < 0 || nrows < 1 || k < 32 || k % 32)
    return fail(SVQ_E_SHAPE, "invalid shape nids=%lld nrows=%lld k=%d",
                (long long)nids, (long long)nrows, k);
  if (out_dtype != SVQ_F32 && out_dtype != SVQ_F16 && out_dtype != SVQ_BF16)
    return fail(SVQ_E_DTYPE, "unsupported out_dtype %d", out_dtype);
  if (nids == 0) return 0;
  if (!q || !s || !ids || !out) return fail(SVQ_E_NULL, "NULL q, s, ids or out");
  if ((int64_t)nids * (k / 32) * 2 > ((int64_t)1 << 36))
    return fail(SVQ_E_RANGE, "too many rows requested");
  if (!aligned(q, qtype == SVQ_Q5_0 ? 4 : 16) || !aligned(s, 2) ||
      !aligned(ids, 8) || !aligned(out, 16))
    return fail(SVQ_E_ALIGN, "misaligned q, ids or out");
  const hipError_t e =
      svq::launch_dequant_rows(q, s, ids, nids, nrows, k, out, qtype, out_dtype,
                               static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "svq_dequant_rows launch");
  return 0;
}

int64_t svq_decode_attention_workspace(int rows, int heads, int kv_heads, int span) {
  if (rows < 1 || kv_heads < 1 || heads < kv_heads || heads % kv_heads != 0 ||
      heads / kv_heads > SVQ_MAX_GROUP || span < 1)
    return fail(SVQ_E_SHAPE, "invalid attention shape rows=%d heads=%d kv_heads=%d span=%d",
                rows, heads, kv_heads, span);
  return svq::attention_workspace_bytes(rows, heads, kv_heads, span);
}

int svq_decode_attention(const uint16_t* qkv, int64_t qkv_stride, const uint16_t* cos,
                         const uint16_t* sin, uint16_t* keys, uint16_t* values,
                         int64_t capacity, const int64_t* position, const uint16_t* bias,
                         int window, int span, uint16_t* out, int rows, int heads, int kv_heads,
                         int head_dim, float scale, void* workspace,
                         int64_t workspace_bytes, void* stream) {
  if (rows < 1 || kv_heads < 1 || heads < kv_heads || heads % kv_heads != 0 ||
      heads / kv_heads > SVQ_MAX_GROUP || head_dim != SVQ_HEAD_DIM || span < 1 ||
      capacity < span || rows * (int64_t)kv_heads > 65535 ||
      qkv_stride < (int64_t)(heads + 2 * kv_heads) * head_dim || qkv_stride % 8 != 0)
    return fail(SVQ_E_SHAPE,
                "invalid attention shape rows=%d heads=%d kv_heads=%d head_dim=%d span=%d "
                "capacity=%lld qkv_stride=%lld",
                rows, heads, kv_heads, head_dim, span, (long long)capacity,
                (long long)qkv_stride);
  if ((int64_t)span * head_dim * 2 >= ((int64_t)1 << 31) ||
      rows * (int64_t)kv_heads * capacity * head_dim >= ((int64_t)1 << 40))
    return fail(SVQ_E_RANGE, "attention cache too large");
  if (!qkv || !keys || !values || !position || !out || !workspace)
    return fail(SVQ_E_NULL, "NULL qkv, keys, values, position, out or workspace");
  if ((cos == nullptr) != (sin == nullptr))
    return fail(SVQ_E_NULL, "cos and sin must both be given or both be NULL");
  if (!aligned(qkv, 16) || !aligned(keys, 16) || !aligned(values, 16) || !aligned(out, 16) ||
      (cos && (!aligned(cos, 16) || !aligned(sin, 16))) || (bias && !aligned(bias, 2)) ||
      !aligned(position, 8) || !aligned(workspace, 256))
    return fail(SVQ_E_ALIGN, "misaligned attention argument");
  const int64_t need = svq::attention_workspace_bytes(rows, heads, kv_heads, span);
  if (workspace_bytes < need)
    return fail(SVQ_E_WORKSPACE, "workspace of %lld bytes, %lld needed",
                (long long)workspace_bytes, (long long)need);
  svq::AttnArgs a{};
  a.qkv = qkv;
  a.qkv_stride = qkv_stride;
  a.cos = cos;
  a.sin = sin;
  a.keys = keys;
  a.values = values;
  a.capacity = capacity;
  a.position = position;
  a.bias = bias;
  a.window = window > 0 ? window : 0;
  a.span = span;
  a.out = out;
  a.kv_heads = kv_heads;
  a.scale = scale;
  a.nchunks = svq::attention_chunks(span);
  a.ml = static_cast<float2*>(workspace);
  a.acc = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                   svq::attention_ml_bytes(rows, heads, span));
  const hipError_t e = svq::launch_decode_attention(a, rows, heads / kv_heads,
                                                    static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "svq_decode_attention launch");
  return 0;
}

int svq_cache_reorder(uint16_t* cache, int64_t planes, int rows, int heads, int64_t capacity,
                      int head_dim, int64_t length, const int64_t* parents, void* stream) {
  if (planes < 1 || rows < 1 || rows > SVQ_MAX_ROWS || heads < 1 || head_dim != SVQ_HEAD_DIM ||
      length < 0 || capacity < length || capacity < 1 || planes * heads > 65535)
    return fail(SVQ_E_SHAPE,
                "invalid cache shape planes=%lld rows=%d heads=%d capacity=%lld head_dim=%d "
                "length=%lld",
                (long long)planes, rows, heads, (long long)capacity, head_dim,
                (long long)length);
  if (length * (head_dim / 8) / 256 >= ((int64_t)1 << 31))
    return fail(SVQ_E_RANGE, "cache reorder length too large");
  if (!cache || !parents) return fail(SVQ_E_NULL, "NULL cache or parents");
  if (!aligned(cache, 16) || !aligned(parents, 8))
    return fail(SVQ_E_ALIGN, "misaligned cache or parents");
  if (length == 0) return 0;
  svq::ReorderArgs a{cache, capacity, length, parents, rows, heads};
  const hipError_t e = svq::launch_cache_reorder(a, planes, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "svq_cache_reorder launch");
  return 0;
}

int svq_beam_select(const float* probs, const float* noise, const float* scores,
                    const int64_t* candidates, int beams, int64_t vocab, int ncand, int draws,
                    const uint8_t* seen_in, uint8_t* seen_out, int64_t seen_pitch,
                    float* running, int64_t* parents, int64_t* tokens, int64_t* tokens_copy,
                    int compact, void* stream) {
  if (beams < 1 || beams > svq::kBeamMaxRows || vocab < 1 || ncand < 1 || ncand > vocab ||
      (int64_t)beams * ncand > svq::kBeamMaxCandidates || draws < 1 || draws > 2 * beams ||
      draws > beams * ncand || seen_pitch < vocab || seen_pitch % 16 != 0)
    return fail(SVQ_E_SHAPE,
                "invalid beam selection beams=%d vocab=%lld candidates=%d draws=%d "
                "seen_pitch=%lld",
                beams, (long long)vocab, ncand, draws, (long long)seen_pitch);
  if ((int64_t)beams * vocab >= ((int64_t)1 << 40) || (int64_t)beams * seen_pitch >= ((int64_t)1 << 40))
    return fail(SVQ_E_RANGE, "beam selection too large");
  if (!probs || !noise || !scores || !candidates || !seen_in || !seen_out || !running ||
      !parents || !tokens)
    return fail(SVQ_E_NULL, "NULL beam selection argument");
  if (!aligned(probs, 4) || !aligned(noise, 4) || !aligned(scores, 4) || !aligned(running, 4) ||
      !aligned(candidates, 8) || !aligned(parents, 8) || !aligned(tokens, 8) ||
      (tokens_copy && !aligned(tokens_copy, 8)) || !aligned(seen_in, 16) || !aligned(seen_out, 16))
    return fail(SVQ_E_ALIGN, "misaligned beam selection argument");
  const int64_t seen_bytes = (int64_t)beams * seen_pitch;
  const uint8_t* out_lo = seen_out;
  if (seen_in < out_lo + seen_bytes && out_lo < seen_in + seen_bytes)
    return fail(SVQ_E_SHAPE, "seen_in and seen_out overlap");
  svq::BeamSelectArgs a{probs,   noise,       scores, candidates, seen_in, seen_out,
                        seen_pitch, running, parents, tokens,     tokens_copy, vocab,
                        beams,   ncand,       draws,  compact != 0};
  if (compact && ncand > svq::kCandMax)
    return fail(SVQ_E_SHAPE, "compact beam selection takes at most %d candidates per beam",
                svq::kCandMax);
  const hipError_t e = svq::launch_beam_select(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "svq_beam_select launch");
  return 0;
}

int64_t svq_beam_candidates_workspace(int beams, int vocab, int kc) {
  if (beams < 1 || beams > svq::kBeamMaxRows || vocab < 1 || vocab > svq::kCandMaxVocab ||
      kc < 1 || kc > svq::kCandMax || kc > vocab)
    return fail(SVQ_E_SHAPE, "invalid beam candidates beams=%d vocab=%d kc=%d", beams, vocab, kc);
  return svq::beam_candidates_workspace(beams, vocab, kc);
}

int svq_beam_candidates(const uint16_t* logits, const uint8_t* seen, int64_t seen_pitch,
                        const float* running, int beams, int vocab, int k, int kc, int keep,
                        float penalty, float temperature, double top_p, int64_t* candidates,
                        float* scores, float* probs, int64_t* status, void* workspace,
                        int64_t workspace_bytes, void* stream) {
  if (beams < 1 || beams > svq::kBeamMaxRows || vocab < 1 || vocab > svq::kCandMaxVocab ||
      k < 1 || kc < k || kc > svq::kCandMax || kc > vocab || keep < 0 || keep > kc ||
      seen_pitch < vocab || seen_pitch % 16 != 0)
    return fail(SVQ_E_SHAPE,
                "invalid beam candidates beams=%d vocab=%d k=%d kc=%d keep=%d seen_pitch=%lld",
                beams, vocab, k, kc, keep, (long long)seen_pitch);
  if (!(temperature > 0.0f) || !(penalty > 0.0f) || !(top_p >= 0.0 && top_p <= 1.0))
    return fail(SVQ_E_SHAPE, "invalid temperature %g, penalty %g or top_p %g",
                (double)temperature, (double)penalty, (double)top_p);
  if (!logits || !seen || !running || !candidates || !scores || !probs || !status || !workspace)
    return fail(SVQ_E_NULL, "NULL beam candidates argument");
  if (!aligned(logits, 2) || !aligned(running, 4) || !aligned(candidates, 8) ||
      !aligned(scores, 4) || !aligned(probs, 4) || !aligned(status, 8) || !aligned(workspace, 8))
    return fail(SVQ_E_ALIGN, "misaligned beam candidates argument");
  const int64_t need = svq::beam_candidates_workspace(beams, vocab, kc);
  if (workspace_bytes < need)
    return fail(SVQ_E_WORKSPACE, "workspace of %lld bytes, %lld needed",
                (long long)workspace_bytes, (long long)need);
  svq::BeamCandArgs a{};
  a.logits = logits;
  a.seen = seen;
  a.seen_pitch = seen_pitch;
  a.running = running;
  a.candidates = candidates;
  a.scores = scores;
  a.probs = probs;
  a.status = status;
  a.vocab = vocab;
  a.beams = beams;
  a.k = k;
  a.kc = kc;
  a.keep = keep;
  a.penalty = penalty;
  a.temperature = temperature;
  a.top_p_cut = (float)(1.0 - top_p);  // torch compares with the fp32 rounding of 1 - top_p
  a.use_top_p = top_p < 1.0;
  a.workspace = workspace;
  const hipError_t e = svq::launch_beam_candidates(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "svq_beam_candidates launch");
  return 0;
}

}  // extern "C"
