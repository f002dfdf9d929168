// Instantiation table of gemm_stream_kernel (W-resident streaming GEMM).
#pragma once

#include "capi.hpp"
#include "gemm_dispatch.hpp"
#include "gemm_stream.hpp"

namespace clarus {

// k-steps of 32 held in registers per 16-pixel block, and the prefetch depth, per A dtype
constexpr int stream_ks_for(int64_t k, int ta) {
  return k <= 64 ? 2 : k <= 128 ? 4 : (k <= 256 && ta == DT_BF16) ? 8 : 0;
}
template <int NB, bool GATE, int OPM, int TA, int KS, bool X2>
void launch_stream_one(const GemmP& p, dim3 grid_max, hipStream_t s, int) {
  constexpr int lds = stream_lds_bytes(NB, GATE, KS, OPM);
  auto fn = &gemm_stream_kernel<NB, GATE, OPM, TA, KS, X2>;
  static const int per_cu = [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024);
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(fn), 256, lds) != hipSuccess ||
        n < 1)
      n = 1;
    return n;
  }();
  // every workgroup resident: 256 CUs x per_cu, split over the channel tiles and batch
  const int64_t blocks16 = cdiv(p.m, 16);
  int64_t gx = ((int64_t)device_cus() * per_cu) / ((int64_t)grid_max.y * grid_max.z);
  if (gx < 1) gx = 1;
  const int64_t need = cdiv(blocks16, 4);  // one 16-pixel block per wave at least
  if (gx > need) gx = need;
  if (gx > 8) gx = gx / 8 * 8;  // keep channel tiles of a pixel range on one XCD
  hipLaunchKernelGGL(fn, dim3((unsigned)gx, grid_max.y, grid_max.z), dim3(256), lds, s, p);
}

GemmLaunch pick_gemm_stream_nogate(int nb, int opm, int ta, int ks, bool x2);
GemmLaunch pick_gemm_stream_gate(int nb, int opm, int ta, int ks, bool x2);
inline GemmLaunch pick_gemm_stream(int nb, bool gate, int opm, int ta, int ks, bool x2) {
  return gate ? pick_gemm_stream_gate(nb, opm, ta, ks, x2) : pick_gemm_stream_nogate(nb, opm, ta, ks, x2);
}

}  // namespace clarus
