// Instantiation table of gemm_kernel: tile ids and the per-addressing-mode pickers.
#pragma once

#include "gemm_kernel.hpp"

namespace clarus {

using GemmLaunch = void (*)(const GemmP&, dim3, hipStream_t, int);

// tile id -> (NB, PB): TN = 16 * NB output channels, TP = 64 * PB pixels per workgroup
constexpr int kTileNB[] = {1, 2, 4, 4, 4, 8, 8};
constexpr int kTilePB[] = {4, 4, 1, 2, 4, 1, 2};
constexpr int kNumTiles = 7;

// nbuf = 1 when K fits one chunk (W resident), 2 for the double-buffered K loop
template <int NB, int PB, bool GATE, int OPM, int TA, int AM, int KC>
void launch_gemm_one(const GemmP& p, dim3 grid, hipStream_t s, int nbuf) {
  static const bool attr_set = [] {
    // dynamic LDS above 64 KiB must be allowed explicitly (gfx950 has 160 KiB per CU)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_kernel<NB, PB, GATE, OPM, TA, AM, KC>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    return true;
  }();
  (void)attr_set;
  const size_t lds = gemm_epi_bytes(NB) + (size_t)nbuf * gemm_wbuf_bytes(NB, GATE, OPM, KC);
  hipLaunchKernelGGL((gemm_kernel<NB, PB, GATE, OPM, TA, AM, KC>), grid, dim3(256), lds, s, p);
}

#define CLARUS_TILE_SWITCH(TILE, F) \
  switch (TILE) {                   \
    case 0: return F(1, 4);         \
    case 1: return F(2, 4);         \
    case 2: return F(4, 1);         \
    case 3: return F(4, 2);         \
    case 4: return F(4, 4);         \
    case 5: return F(8, 1);         \
    case 6: return F(8, 2);         \
    default: return nullptr;        \
  }

// operand mode x A dtype combos: (OPM_BF16, bf16), (OPM_SPLIT, bf16|f32), (OPM_F32, bf16|f32)
GemmLaunch pick_gemm_rows_nogate(int tile, int opm, int ta);
GemmLaunch pick_gemm_rows_gate(int tile, int opm, int ta);
inline GemmLaunch pick_gemm_rows(int tile, bool gate, int opm, int ta) {
  return gate ? pick_gemm_rows_gate(tile, opm, ta) : pick_gemm_rows_nogate(tile, opm, ta);
}
GemmLaunch pick_gemm_s2d(int tile, int opm, int ta);
GemmLaunch pick_gemm_conv(int tile, int opm, int ta);

// K chunk staged in LDS per operand mode
constexpr int kc_for(int opm) { return opm == OPM_F32 ? 64 : 128; }

}  // namespace clarus
