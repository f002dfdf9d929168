// conv_halo_kernel instantiations and launcher.
#include "capi.hpp"
#include "conv_halo.hpp"
#include "gemm_lds_dispatch.hpp"

namespace clarus {

namespace {

constexpr int kLdsMax = 160 * 1024;

template <int TR, bool UP2, int STAGES>
void launch_one(GemmP& p, hipStream_t s) {
  auto fn = &conv_halo_kernel<TR, UP2, STAGES>;
  const int lds = conv_halo_lds_bytes(TR, p.cin, UP2, STAGES);
  static const bool attr = (hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                                hipFuncAttributeMaxDynamicSharedMemorySize, kLdsMax),
                            true);
  (void)attr;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(fn), 512, lds) !=
          hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  const int64_t H = (int64_t)p.h << (UP2 ? 1 : 0), W = (int64_t)p.w << (UP2 ? 1 : 0);
  const int64_t ptiles = (p.m / (H * W)) * cdiv(H, (int64_t)HaloGeom<UP2>::th) * cdiv(W, CH_TW);
  const int64_t ncol = cdiv(p.n, TR);
  int64_t per_col = (int64_t)device_cus() * per_cu / ncol;  // persistent: every workgroup resident
  if (per_col > ptiles) per_col = ptiles;
  per_col = per_col < 8 ? 8 : per_col / 8 * 8;  // a multiple of 8: the kernel deals tiles per XCD
  hipLaunchKernelGGL(fn, dim3((unsigned)(per_col * ncol)), dim3(512), lds, s, p);
}

template <int TR, bool UP2>
bool launch_tr(GemmP& p, hipStream_t s) {
  if (conv_halo_lds_bytes(TR, p.cin, UP2, 3) <= kLdsMax) launch_one<TR, UP2, 3>(p, s);
  else if (conv_halo_lds_bytes(TR, p.cin, UP2, 2) <= kLdsMax) launch_one<TR, UP2, 2>(p, s);
  else return false;
  return true;
}

}  // namespace

bool launch_conv_halo(GemmP& p, hipStream_t s) {
  // chunk offsets must stay inside the 1 KiB zero page: (cin / 32 - 1) * 64 + 64 <= 1024
  if (p.cin % CH_KC != 0 || p.cin > 448) return false;
  const bool up2 = p.up2 != 0;
  // 64-channel tiles where the resident weights fit, else 32 (16 for at most 16 channels)
  const bool tr64 = p.n >= 64 && conv_halo_lds_bytes(64, p.cin, up2, 2) <= kLdsMax;
  if (tr64) return up2 ? launch_tr<64, true>(p, s) : launch_tr<64, false>(p, s);
  if (p.n <= 16 && !up2) return launch_tr<16, false>(p, s);  // narrow outputs: half the MFMA work of 32
  return up2 ? launch_tr<32, true>(p, s) : launch_tr<32, false>(p, s);
}

}  // namespace clarus
