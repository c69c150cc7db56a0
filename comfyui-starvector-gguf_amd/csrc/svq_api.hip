// C ABI of libsvq.so (declared in include/svq.h): argument validation, launch
// shape selection and error reporting. Every argument check runs before any
// HIP call, so rejected calls need no GPU.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "../../include/svq.h"
#include "svq_launch.h"

namespace {

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

// Launch-shape overrides for tuning sweeps: SVQ_LG_G (log2 lanes per row),
// SVQ_ROWS (rows per lane group, 1 or 2), SVQ_LDS_KB (LDS budget per
// workgroup). Read once per process.
struct Tuning {
  int lg_g = -1;
  int rows = 0;
  int lds_kb = 40;
};

const Tuning& tuning() {
  static Tuning t;
  static std::once_flag once;
  std::call_once(once, [] {
    if (const char* v = getenv("SVQ_LG_G")) t.lg_g = atoi(v);
    if (const char* v = getenv("SVQ_ROWS")) t.rows = atoi(v);
    if (const char* v = getenv("SVQ_LDS_KB")) t.lds_kb = atoi(v);
    if (t.lg_g > 6) t.lg_g = 6;
    if (t.rows != 0 && t.rows != 1 && t.rows != 2) t.rows = 0;
    if (t.lds_kb < 4 || t.lds_kb > 64) t.lds_kb = 40;
  });
  return t;
}

svq::GemvShape choose_shape(int m, int n, int k, int qtype) {
  const Tuning& tu = tuning();
  svq::GemvShape sh;
  sh.m = m;
  const int units = (k / 32) * svq::units_per_block(qtype);
  // Lanes per row: as many as keep >= 8 units per lane, at most a wave.
  int lg_g = 6;
  while (lg_g > 0 && (units >> lg_g) < 8) --lg_g;
  if (tu.lg_g >= 0) lg_g = tu.lg_g;
  sh.lg_g = lg_g;
  const int row_groups_per_wave = 64 >> lg_g;
  // Two rows per lane group halve LDS activation traffic for M >= 2 when
  // the grid still has >= 2 workgroups per CU of a 256-CU part.
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

}  // namespace

extern "C" {

int svq_abi_version(void) { return SVQ_ABI_VERSION; }

const char* svq_last_error(void) { return g_error; }

int svq_gemv(const void* x, const uint8_t* q, const uint16_t* s,
             const uint16_t* bias, void* y, int m, int n, int k, int qtype,
             int y_dtype, void* stream) {
  if (!valid_qtype(qtype)) return fail(SVQ_E_QTYPE, "unsupported qtype %d", qtype);
  if (m < 1 || m > SVQ_MAX_ROWS)
    return fail(SVQ_E_SHAPE, "m=%d outside 1..%d", m, SVQ_MAX_ROWS);
  if (n < 1 || k < 32 || k % 32)
    return fail(SVQ_E_SHAPE, "invalid matrix dimensions n=%d k=%d", n, k);
  if (k > (1 << 24) || n > (1 << 30))
    return fail(SVQ_E_RANGE, "n=%d k=%d exceeds the supported range", n, k);
  if (!x || !q || !s || !y) return fail(SVQ_E_NULL, "NULL x, q, s or y");
  if (y_dtype != SVQ_F16 && y_dtype != SVQ_F32)
    return fail(SVQ_E_DTYPE, "y_dtype %d is not SVQ_F16 or SVQ_F32", y_dtype);
  if (!aligned(x, 16) || !aligned(q, qtype == SVQ_Q5_0 ? 4 : 16) ||
      !aligned(s, 2) || (bias && !aligned(bias, 2)) ||
      !aligned(y, y_dtype == SVQ_F32 ? 4 : 2))
    return fail(SVQ_E_ALIGN, "misaligned pointer (x and q need 16 bytes)");
  // Per-wave 32-bit offsets: up to 128 rows of payload.
  if ((uint64_t)(k / 32) * payload_bytes(qtype) * 128 >= (1ull << 32))
    return fail(SVQ_E_RANGE, "row of %d weights too long", k);
  const svq::GemvShape sh = choose_shape(m, n, k, qtype);
  svq::GemvArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.q = q;
  a.s = s;
  a.bias = bias;
  a.y = y;
  a.n = n;
  a.k = k;
  a.lg_g = sh.lg_g;
  a.chunk_units = sh.chunk_units;
  a.y_f32 = y_dtype == SVQ_F32;
  const hipError_t e =
      svq::launch_gemv(a, sh, qtype, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "svq_gemv launch");
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

}  // extern "C"
