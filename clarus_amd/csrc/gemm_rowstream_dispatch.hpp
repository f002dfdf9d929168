// Launcher of gemm_rowstream_kernel (streaming GEMM with an LDS ring per wave).
#pragma once

#include "gemm_kernel.hpp"

namespace clarus {

// k-steps of 32 per row for the ring kernel (0: K too long for it)
int rowstream_ks_for(int64_t k, int ta);

// Launches the kernel for p (AM_ROWS; no prologue, or LN / RMS / the bf16 TLC map multiply on
// split operands with batch 1; row or pixel-shuffle output; p.ptiles unused). nb: channel
// blocks of 16 per workgroup (4 or 8); res / rdt: a residual of that dtype (not with gate; the
// host checks 16-byte rows and n % (16 / residual element size) == 0). Returns false when no
// instantiation matches.
bool launch_gemm_rowstream(const GemmP& p, int nb, bool gate, int opm, int ta, int ks, bool res, int rdt,
                           int64_t batch, hipStream_t s);

}  // namespace clarus
