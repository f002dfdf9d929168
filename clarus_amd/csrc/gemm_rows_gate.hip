// gemm_kernel instantiations for NHWC row operands with SimpleGate (B holds 2N columns; two
// accumulator sets multiplied in the epilogue).
#include "gemm_dispatch.hpp"

namespace clarus {

#define G_BF(nb, pb) (&launch_gemm_one<nb, pb, GATE_, OPM_BF16, DT_BF16, AM_ROWS, 128>)
#define G_SB(nb, pb) (&launch_gemm_one<nb, pb, GATE_, OPM_SPLIT, DT_BF16, AM_ROWS, 128>)
#define G_SF(nb, pb) (&launch_gemm_one<nb, pb, GATE_, OPM_SPLIT, DT_F32, AM_ROWS, 128>)
#define G_FB(nb, pb) (&launch_gemm_one<nb, pb, GATE_, OPM_F32, DT_BF16, AM_ROWS, 64>)
#define G_FF(nb, pb) (&launch_gemm_one<nb, pb, GATE_, OPM_F32, DT_F32, AM_ROWS, 64>)

template <bool GATE_>
static GemmLaunch pick(int tile, int opm, int ta) {
  if (opm == OPM_BF16) {
    if (ta != DT_BF16) return nullptr;
    CLARUS_TILE_SWITCH(tile, G_BF)
  }
  if (opm == OPM_SPLIT) {
    if (ta == DT_BF16) { CLARUS_TILE_SWITCH(tile, G_SB) }
    CLARUS_TILE_SWITCH(tile, G_SF)
  }
  if (opm == OPM_F32) {
    if (ta == DT_BF16) { CLARUS_TILE_SWITCH(tile, G_FB) }
    CLARUS_TILE_SWITCH(tile, G_FF)
  }
  return nullptr;
}

GemmLaunch pick_gemm_rows_gate(int tile, int opm, int ta) { return pick<true>(tile, opm, ta); }

}  // namespace clarus
