// gemm_rowstream_kernel instantiations and launcher (streaming GEMM with an LDS ring per wave).
#include "capi.hpp"
#include "gemm_rowstream.hpp"
#include "gemm_rowstream_dispatch.hpp"

namespace clarus {

namespace {

template <int NB, bool GATE, int OPM, int TA, int KS, bool RES, int RDT, bool X2>
void launch_one(const GemmP& p, unsigned ny, unsigned nz, hipStream_t s) {
  constexpr int lds = rowstream_lds_bytes(NB, GATE, KS, OPM, TA, RDT, RES, X2);
  constexpr int nw = rowstream_waves(NB, GATE, KS, OPM, TA, RDT, RES, X2);
  static_assert(lds <= 160 * 1024, "LDS budget");
  auto fn = &gemm_rowstream_kernel<NB, GATE, OPM, TA, KS, RES, RDT, X2>;
  static const int per_cu = [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024);
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(fn), 64 * nw, lds) !=
            hipSuccess ||
        n < 1)
      n = 1;
    return n;
  }();
  // every workgroup resident: 256 CUs x per_cu, split over the channel tiles and batch; a
  // multiple of 8 keeps the channel tiles of a pixel range on one XCD
  const int64_t blocks = cdiv(p.m, RS_BP);
  int64_t gx = ((int64_t)device_cus() * per_cu) / ((int64_t)ny * nz);
  if (gx < 1) gx = 1;
  const int64_t need = cdiv(blocks, nw);
  if (gx > need) gx = need;
  if (gx > 8) gx = gx / 8 * 8;
  hipLaunchKernelGGL(fn, dim3((unsigned)gx, ny, nz), dim3(64 * nw), lds, s, p);
}

using RsLaunch = void (*)(const GemmP&, unsigned, unsigned, hipStream_t);

template <int NB, bool GATE, int OPM, int TA, int KS, bool RES, int RDT, bool X2>
constexpr RsLaunch one_if_fits() {
  if constexpr (rowstream_depth(NB, GATE, KS, OPM, TA, RDT, RES, X2) >= 2)
    return &launch_one<NB, GATE, OPM, TA, KS, RES, RDT, X2>;
  else
    return nullptr;
}

template <int NB, bool GATE, int OPM, int TA, int KS, bool X2>
RsLaunch pick_res(bool res, int rdt) {
  if (!res) return one_if_fits<NB, GATE, OPM, TA, KS, false, DT_BF16, X2>();
  if constexpr (GATE) {
    return nullptr;
  } else {
    return rdt == DT_BF16 ? one_if_fits<NB, false, OPM, TA, KS, true, DT_BF16, X2>()
                          : one_if_fits<NB, false, OPM, TA, KS, true, DT_F32, X2>();
  }
}

template <int NB, bool GATE, int OPM, int TA, bool X2>
RsLaunch pick_ks(int ks, bool res, int rdt) {
  switch (ks) {
    case 1: return pick_res<NB, GATE, OPM, TA, 1, X2>(res, rdt);
    case 2: return pick_res<NB, GATE, OPM, TA, 2, X2>(res, rdt);
    case 4:
      if constexpr (TA == DT_BF16) return pick_res<NB, GATE, OPM, TA, 4, X2>(res, rdt);
      return nullptr;
    default: return nullptr;
  }
}

// operand modes: bf16 A without prologue; fp32 A split into hi + lo (bf16 W) or fp32 products
// (fp32 W); bf16 A with a prologue (LN / RMS, or the map multiply with x2) split into hi + lo or
// rounded once to bf16
template <int NB, bool GATE>
RsLaunch pick_mode(int opm, int ta, int ks, bool res, int rdt, bool pro, bool x2) {
  if (opm == OPM_BF16 && ta == DT_BF16 && !pro) return pick_ks<NB, GATE, OPM_BF16, DT_BF16, false>(ks, res, rdt);
  if (opm == OPM_SPLIT && ta == DT_F32 && !x2) return pick_ks<NB, GATE, OPM_SPLIT, DT_F32, false>(ks, res, rdt);
  if (opm == OPM_F32 && ta == DT_F32 && !pro) return pick_ks<NB, GATE, OPM_F32, DT_F32, false>(ks, res, rdt);
  if (opm == OPM_SPLIT && ta == DT_BF16 && pro)
    return x2 ? pick_ks<NB, GATE, OPM_SPLIT, DT_BF16, true>(ks, res, rdt)
              : pick_ks<NB, GATE, OPM_SPLIT, DT_BF16, false>(ks, res, rdt);
  if (opm == OPM_ROUND && ta == DT_BF16 && pro)
    return x2 ? pick_ks<NB, GATE, OPM_ROUND, DT_BF16, true>(ks, res, rdt)
              : pick_ks<NB, GATE, OPM_ROUND, DT_BF16, false>(ks, res, rdt);
  return nullptr;
}

}  // namespace

int rowstream_ks_for(int64_t k, int ta) {
  if (k <= 32) return 1;
  if (k <= 64) return 2;
  if (k <= 128 && ta == DT_BF16) return 4;
  return 0;
}

bool launch_gemm_rowstream(const GemmP& p, int nb, bool gate, int opm, int ta, int ks, bool res, int rdt,
                           int64_t batch, hipStream_t s) {
  const bool pro = p.pro != PRO_NONE, x2 = p.pro == PRO_MUL;
  RsLaunch fn = nullptr;
  if (nb == 4)
    fn = gate ? pick_mode<4, true>(opm, ta, ks, res, rdt, pro, x2) : pick_mode<4, false>(opm, ta, ks, res, rdt, pro, x2);
  else if (nb == 8)
    fn = gate ? pick_mode<8, true>(opm, ta, ks, res, rdt, pro, x2) : pick_mode<8, false>(opm, ta, ks, res, rdt, pro, x2);
  if (!fn) return false;
  fn(p, (unsigned)cdiv(p.n, 16 * nb), (unsigned)batch, s);
  return true;
}

}  // namespace clarus
