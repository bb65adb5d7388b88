// One wave per item, shallow-pipeline kernels for short items (their lower
// register count admits more waves per SIMD).

#include "scan_item.h"

namespace asc {

const void* item_fwd_short_kernel(int dtype, int dirs, bool aln, bool wa) {
  switch (dtype) {
    case ASC_F32: return pick_fwd<IoF32, kFwdShallow>(dirs, aln, wa);
    case ASC_F16: return pick_fwd<IoF16, kFwdShallow>(dirs, aln, wa);
    default: return pick_fwd<IoBF16, kFwdShallow>(dirs, aln, wa);
  }
}

const void* item_bwd_short_kernel(int dtype, int dirs, bool aln, bool dyc) {
  switch (dtype) {
    case ASC_F32: return pick_bwd<IoF32, kBwdShallow>(dirs, aln, dyc);
    case ASC_F16: return pick_bwd<IoF16, kBwdShallow>(dirs, aln, dyc);
    default: return pick_bwd<IoBF16, kBwdShallow>(dirs, aln, dyc);
  }
}

}  // namespace asc
