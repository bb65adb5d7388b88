// One wave per item, shallow-pipeline kernels for short items (their lower
// register count admits more waves per SIMD).

#include "scan_item.h"

namespace asc {
namespace {

// Pipeline depth (sub-tiles per block) of the short-item kernels.
constexpr int kFwdUnrollShort = 2, kBwdUnrollShort = 1;

}  // namespace

const void* item_fwd_short_kernel(int dtype, int dirs, bool aln, bool wa) {
  switch (dtype) {
    case ASC_F32: return pick_fwd<IoF32, kFwdUnrollShort>(dirs, aln, wa);
    case ASC_F16: return pick_fwd<IoF16, kFwdUnrollShort>(dirs, aln, wa);
    default: return pick_fwd<IoBF16, kFwdUnrollShort>(dirs, aln, wa);
  }
}

const void* item_bwd_short_kernel(int dtype, int dirs, bool aln, bool dyc) {
  switch (dtype) {
    case ASC_F32: return pick_bwd<IoF32, kBwdUnrollShort>(dirs, aln, dyc);
    case ASC_F16: return pick_bwd<IoF16, kBwdUnrollShort>(dirs, aln, dyc);
    default: return pick_bwd<IoBF16, kBwdUnrollShort>(dirs, aln, dyc);
  }
}

}  // namespace asc
