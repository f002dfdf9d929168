// gemm_lds_kernel instantiations and launcher.
#include "capi.hpp"
#include "gemm_dma.hpp"
#include "gemm_mfma32.hpp"
#include "gemm_big.hpp"
#include "gemm_lds.hpp"
#include "gemm_lds_dispatch.hpp"

namespace clarus {

namespace {

constexpr int kLdsKC = 32;

template <int OPM, int TA, bool GATE, bool X2>
void launch_one(GemmP& p, hipStream_t s) {
  constexpr int lds = lt_lds_bytes(kLdsKC, OPM);
  auto fn = &gemm_lds_kernel<OPM, TA, GATE, X2, kLdsKC>;
  static const int per_cu = [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024);
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(fn), 256, lds) != hipSuccess ||
        n < 1)
      n = 1;
    return n;
  }();
  p.ptiles = cdiv(p.m, LT_P);
  const int64_t tiles = p.ptiles * cdiv(p.n, LT_R / (GATE ? 2 : 1));
  // persistent: every workgroup resident, a multiple of 8 so each XCD gets the same number
  int64_t gx = (int64_t)device_cus() * per_cu;
  const int64_t need = cdiv(tiles, 8) * 8;
  if (gx > need) gx = need;
  hipLaunchKernelGGL(fn, dim3((unsigned)gx), dim3(256), lds, s, p);
}

template <bool GATE>
void launch_dma(GemmP& p, hipStream_t s) {
  constexpr int lds = dma_lds_bytes();
  auto fn = &gemm_dma_kernel<GATE>;
  static const int per_cu = [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024);
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(fn), 256, lds) != hipSuccess ||
        n < 1)
      n = 1;
    return n;
  }();
  p.ptiles = cdiv(p.m, DMA_P);
  const int64_t tiles = p.ptiles * cdiv(p.n, DMA_R / (GATE ? 2 : 1));
  int64_t gx = (int64_t)device_cus() * per_cu;
  const int64_t need = cdiv(tiles, 8) * 8;
  if (gx > need) gx = need;
  hipLaunchKernelGGL(fn, dim3((unsigned)gx), dim3(256), lds, s, p);
}

template <bool GATE>
void launch_m32(GemmP& p, hipStream_t s) {
  auto fn = &gemm_mfma32_kernel<GATE>;
  static const int per_cu = [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024);
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(fn), 256, M32_LDS) !=
            hipSuccess ||
        n < 1)
      n = 1;
    return n;
  }();
  p.ptiles = cdiv(p.m, M32_P);
  const int64_t tiles = p.ptiles * cdiv(p.n, M32_R / (GATE ? 2 : 1));
  int64_t gx = (int64_t)device_cus() * per_cu;
  const int64_t need = cdiv(tiles, 8) * 8;
  if (gx > need) gx = need;
  hipLaunchKernelGGL(fn, dim3((unsigned)gx), dim3(256), M32_LDS, s, p);
}

template <bool GATE, int WP>
void launch_big(GemmP& p, hipStream_t s) {
  using C = BigCfg<WP>;
  auto fn = &gemm_big_kernel<GATE, WP>;
  static const int per_cu = [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024);
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(fn), C::NT, C::LDS) !=
            hipSuccess ||
        n < 1)
      n = 1;
    return n;
  }();
  p.ptiles = cdiv(p.m, C::P);
  const int64_t tiles = p.ptiles * cdiv(p.n, BIG_R / (GATE ? 2 : 1));
  int64_t gx = (int64_t)device_cus() * per_cu;
  const int64_t need = cdiv(tiles, 8) * 8;
  if (gx > need) gx = need;
  hipLaunchKernelGGL(fn, dim3((unsigned)gx), dim3(C::NT), C::LDS, s, p);
}

}  // namespace

int64_t gemm_big_tiles(int64_t m, int64_t n, bool gate, int wp) {
  return cdiv(m, 128 * wp) * cdiv(n, BIG_R / (gate ? 2 : 1));
}

void launch_gemm_big(GemmP& p, bool gate, int wp, hipStream_t s) {
  if (wp == 2) {
    if (gate) launch_big<true, 2>(p, s);
    else launch_big<false, 2>(p, s);
  } else {
    if (gate) launch_big<true, 1>(p, s);
    else launch_big<false, 1>(p, s);
  }
}

void launch_gemm_m32(GemmP& p, bool gate, hipStream_t s) {
  if (gate) launch_m32<true>(p, s);
  else launch_m32<false>(p, s);
}

void launch_gemm_dma(GemmP& p, bool gate, hipStream_t s) {
  if (gate) launch_dma<true>(p, s);
  else launch_dma<false>(p, s);
}

bool launch_gemm_lds(GemmP& p, bool gate, int opm, int ta, bool x2, hipStream_t s) {
  if (opm == OPM_BF16) {
    if (ta != DT_BF16 || x2) return false;
    if (gate) launch_one<OPM_BF16, DT_BF16, true, false>(p, s);
    else launch_one<OPM_BF16, DT_BF16, false, false>(p, s);
    return true;
  }
  if (opm != OPM_SPLIT) return false;
#define LDS_SPLIT(TA)                                                  \
  if (gate) {                                                          \
    if (x2) launch_one<OPM_SPLIT, TA, true, true>(p, s);               \
    else launch_one<OPM_SPLIT, TA, true, false>(p, s);                 \
  } else {                                                             \
    if (x2) launch_one<OPM_SPLIT, TA, false, true>(p, s);              \
    else launch_one<OPM_SPLIT, TA, false, false>(p, s);                \
  }
  if (ta == DT_BF16) { LDS_SPLIT(DT_BF16) } else { LDS_SPLIT(DT_F32) }
#undef LDS_SPLIT
  return true;
}

}  // namespace clarus
