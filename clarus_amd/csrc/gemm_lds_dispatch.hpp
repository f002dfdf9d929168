// Launcher of gemm_lds_kernel (pipelined LDS-tiled GEMM for long-K row operands).
#pragma once

#include "gemm_epi32.hpp"

namespace clarus {

// Launches the kernel for p (AM_ROWS, batch 1, p.ptiles unset). Returns false when no
// instantiation matches (operand mode, A dtype, gate, second prologue operand).
bool launch_gemm_lds(GemmP& p, bool gate, int opm, int ta, bool x2, hipStream_t s);

// Launches gemm_dma_kernel for p (AM_ROWS, batch 1, bf16 A and W, no prologue, K % 32 == 0).
void launch_gemm_dma(GemmP& p, bool gate, hipStream_t s);

// Launches gemm_mfma32_kernel for p (AM_ROWS, batch 1, bf16 A and W, no prologue, K % 64 == 0,
// a pixel-shuffle quadrant a multiple of 16 channels, epi32_tables_fit(n, gate)).
void launch_gemm_m32(GemmP& p, bool gate, hipStream_t s);

// Launches gemm_big_kernel for p (same operands as launch_gemm_m32): 256 W^T rows x 128 * wp
// pixels per tile, wp in {1, 2}.
void launch_gemm_big(GemmP& p, bool gate, int wp, hipStream_t s);
// number of gemm_big_kernel tiles of a problem
int64_t gemm_big_tiles(int64_t m, int64_t n, bool gate, int wp);

// gemm_slice_kernel (bf16 A and W rows, no prologue / gate / act / residual, row output): K of
// 128, 256 or 512, N % 64 == 0, 16-byte output vectors. launch_gemm_slice returns false when p
// does not fit.
bool gemm_slice_fits(const GemmP& p);
bool launch_gemm_slice(const GemmP& p, hipStream_t s);

// Launches conv_halo_kernel for p (bf16 x and weights, cin % 32 == 0, row output). Returns
// false when the resident weights of even a 32-channel tile do not fit in LDS.
bool launch_conv_halo(GemmP& p, hipStream_t s);

// output channels per lane run (the run must divide a pixel-shuffle quadrant)
constexpr int gemm_lds_run(bool gate) { return gate ? 8 : 16; }
constexpr int kGemmM32Run = 16;

}  // namespace clarus
