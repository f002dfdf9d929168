// gemm_stream_kernel instantiations, SimpleGate = false.
#include "gemm_stream_dispatch.hpp"

namespace clarus {

#define S_ONE(NB, OPM, TA, KS, X2) (&launch_stream_one<NB, false, OPM, TA, KS, X2>)
#define S_KS(NB, OPM, TA, X2)                     \
  switch (ks) {                                   \
    case 2: return S_ONE(NB, OPM, TA, 2, X2);     \
    case 4: return S_ONE(NB, OPM, TA, 4, X2);     \
    case 8: if (TA == DT_BF16) return S_ONE(NB, OPM, TA, 8, X2); return nullptr; \
    default: return nullptr;                      \
  }
#define S_MODES(NB)                                                  \
  if (opm == OPM_BF16 && ta == DT_BF16 && !x2) { S_KS(NB, OPM_BF16, DT_BF16, false) } \
  if (opm == OPM_SPLIT && ta == DT_BF16) {                           \
    if (x2) { S_KS(NB, OPM_SPLIT, DT_BF16, true) }                    \
    S_KS(NB, OPM_SPLIT, DT_BF16, false)                              \
  }                                                                  \
  if (opm == OPM_SPLIT && ta == DT_F32 && ks <= 4) {                 \
    if (x2) { S_KS(NB, OPM_SPLIT, DT_F32, true) }                     \
    S_KS(NB, OPM_SPLIT, DT_F32, false)                               \
  }                                                                  \
  if (opm == OPM_F32 && ta == DT_F32 && ks <= 4 && !x2) {             \
    S_KS(NB, OPM_F32, DT_F32, false)                                 \
  }                                                                  \
  return nullptr;

GemmLaunch pick_gemm_stream_nogate(int nb, int opm, int ta, int ks, bool x2) {
  if (nb == 4) { S_MODES(4) }
  if (nb == 8) { S_MODES(8) }
  return nullptr;
}

}  // namespace clarus
