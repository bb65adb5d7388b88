// One wave per (segment, channel) item (short segments, most fp16/bf16
// problems and the gate-product output): the deep-pipeline kernels and the
// launchers, which pick the pipeline depth from the mean segment length.

#include "scan_item.h"

namespace asc {
namespace {

// Short items: a mean segment of at most 4 sub-tiles (fp32 backward: 3,
// fp16/bf16 backward: 6).  Their waves run the shallow-pipeline kernels,
// whose lower register count admits more waves per SIMD (fp32 forward 93 -> 57 VGPRs,
// bf16 backward 125 -> 96).  Measured on MI355X, uniform segments of
// C=1024 rows: bf16 1024 elements 4.9 / 5.6 -> 6.2 / 6.2 TB/s (fwd / bwd),
// 512 elements 3.4 / 4.3 -> 4.3 / 5.0; fp32 600 elements 5.7 / 5.3 ->
// 6.2 / 5.5; longer segments keep the deep pipeline (bf16 4096 elements:
// 6.3 / 6.1 against 6.0 / 5.9 shallow).
// fp32 forward: up to 4 sub-tiles.  The deep forward pipeline only starts
// past 4 sub-tiles, and at 4 its registers cost occupancy for nothing (T =
// 1024: 29.8 against 31.0 us; ragged segments of 16-2048 elements: 122 against
// 128 us); the backward is slower shallow at 4 (ragged 500-1500: 246 against
// 242 us) and keeps 3 (shallow up to 5 with the edge loads issued together:
// ragged 500-1500 263.5 against 248.9 us; forward up to 6: no gain).
// fp16/bf16 backward: up to 6 sub-tiles (with the edge sub-tiles' loads
// issued together, the shallow backward's extra waves pay off further:
// ragged 1-5000 bf16 elements 279.9 -> 259.0 us, uniform 3000 93.7 -> 91.1;
// cfg3, a mean of 7.2 sub-tiles, stays deep: 420.9 against 429.7 us
// shallow, and so does the forward, 244.2 against 261.8).
bool short_items(const Geometry& geo, int v, bool bwd) {
  const int64_t mean = geo.T / (geo.S > 0 ? geo.S : 1);
  const int64_t subtiles = v != 4 ? (bwd ? 6 : 4) : (bwd ? 3 : 4);
  return mean <= subtiles * static_cast<int64_t>(kWave) * v;
}

}  // namespace

int item_fwd(FwdParams p, int dtype, int dirs, bool aln, bool wa,
             void* stream) {
  const void* fn = nullptr;
  if (short_items(p.geo, 16 / elem_size(dtype), false)) {
    fn = item_fwd_short_kernel(dtype, dirs, aln, wa);
  } else {
    switch (dtype) {
      case ASC_F32: fn = pick_fwd<IoF32, kFwdDeep>(dirs, aln, wa); break;
      case ASC_F16: fn = pick_fwd<IoF16, kFwdDeep>(dirs, aln, wa); break;
      default: fn = pick_fwd<IoBF16, kFwdDeep>(dirs, aln, wa); break;
    }
  }
  const int64_t items = p.geo.items * p.geo.nbranch;
  return launch(fn, walk_grid(p, (items + kWPB - 1) / kWPB, kWPB), kWPB, p, stream);
}

int item_bwd(BwdParams p, int dtype, int dirs, bool aln, bool dyc,
             void* stream) {
  const void* fn = nullptr;
  if (short_items(p.geo, 16 / elem_size(dtype), true)) {
    fn = item_bwd_short_kernel(dtype, dirs, aln, dyc);
  } else {
    switch (dtype) {
      case ASC_F32: fn = pick_bwd<IoF32, kBwdDeep>(dirs, aln, dyc); break;
      case ASC_F16: fn = pick_bwd<IoF16, kBwdDeep>(dirs, aln, dyc); break;
      default: fn = pick_bwd<IoBF16, kBwdDeep>(dirs, aln, dyc); break;
    }
  }
  const int64_t items = p.geo.items * p.geo.nbranch;
  return launch(fn, walk_grid(p, (items + kWPB - 1) / kWPB, kWPB), kWPB, p, stream);
}

}  // namespace asc
