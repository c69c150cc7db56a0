// Streaming fused GGUF SoA dequantize + GEMV on the 4x4x4 matrix cores: the
// instantiations for M = 5..8 (two A halves per unpacked weight operand).
// The kernel template is in svq_mfma4_kernel.h.
#include "svq_mfma4_kernel.h"

namespace svq {

namespace {

template <int QT>
hipError_t wide_dispatch_m(const GemvArgs& a, bool ln, int m, int rows, int groups, size_t lds,
                           hipStream_t stream, const void** fn) {
  switch (m) {
    case 5: return mfma4_dispatch_r<QT, 5>(a, ln, rows, groups, lds, stream, fn);
    case 6: return mfma4_dispatch_r<QT, 6>(a, ln, rows, groups, lds, stream, fn);
    case 7: return mfma4_dispatch_r<QT, 7>(a, ln, rows, groups, lds, stream, fn);
    case 8: return mfma4_dispatch_r<QT, 8>(a, ln, rows, groups, lds, stream, fn);
  }
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t mfma4_dispatch_wide(const GemvArgs& a, bool ln, int qtype, int m, int rows, int groups,
                               size_t lds, hipStream_t stream, const void** fn) {
  switch (qtype) {
    case 4: return wide_dispatch_m<4>(a, ln, m, rows, groups, lds, stream, fn);
    case 5: return wide_dispatch_m<5>(a, ln, m, rows, groups, lds, stream, fn);
    case 8: return wide_dispatch_m<8>(a, ln, m, rows, groups, lds, stream, fn);
  }
  return hipErrorInvalidValue;
}

}  // namespace svq
