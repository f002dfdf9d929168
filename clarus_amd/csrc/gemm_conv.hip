// gemm_kernel instantiations for the implicit 3x3 convolution A operand (conv3x3, ending).
#include "gemm_dispatch.hpp"

namespace clarus {

#define G_BF(nb, pb) (&launch_gemm_one<nb, pb, false, OPM_BF16, DT_BF16, AM_CONV3, 128>)
#define G_SB(nb, pb) (&launch_gemm_one<nb, pb, false, OPM_SPLIT, DT_BF16, AM_CONV3, 128>)
#define G_SF(nb, pb) (&launch_gemm_one<nb, pb, false, OPM_SPLIT, DT_F32, AM_CONV3, 128>)
#define G_FB(nb, pb) (&launch_gemm_one<nb, pb, false, OPM_F32, DT_BF16, AM_CONV3, 64>)
#define G_FF(nb, pb) (&launch_gemm_one<nb, pb, false, OPM_F32, DT_F32, AM_CONV3, 64>)

GemmLaunch pick_gemm_conv(int tile, int opm, int ta) {
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

}  // namespace clarus
