// Row-layout epilogue of the 32x32x16-MFMA tile kernels, staged through LDS (gfx950).
//
// In the MFMA layout a lane owns 16 consecutive channels of ONE pixel: a 16-byte store
// instruction then writes two separate 16-byte pieces into each of 32 pixel rows, and the
// memory pipeline handles it as ~64 partial-line writes. Measured on the NAFNet level-3 shape
// (14400 x 512 x 1024), the epilogue of a 256 x 256 tile took 12-15 us for 128 KiB, about
// 4 B/clk per CU. This epilogue goes through LDS instead, per 32-pixel block of a wave:
//   1. MFMA layout: + bias (SimpleGate: both halves), act, * scale (from LDS tables), written
//      as fp32 rows of the wave's 64 (gate: 32) channels into 8 KiB of LDS. The 16-byte units
//      of a row are XOR-swizzled by the row index (mod the units per row), so the lanes writing
//      32 rows at one column and the lanes reading one row hit distinct bank groups;
//   2. row layout: 8 lanes (gate: 4) share one pixel, 8 consecutive channels each, so a
//      residual load or an output store instruction covers whole 128-byte (64-byte) row
//      segments of 8 (16) pixels.
// The LDS tables hold bias [G * n] and scale * out_scale [n] for the whole problem, loaded once
// per workgroup (epi32_tables); the kernels take only problems whose tables fit (16 KiB).
#pragma once

#include "gemm_lds.hpp"

namespace clarus {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int EPI32_TABLE_FLOATS = 4096;  // bias (G regions) + scale (1 region), each align16(n)
constexpr int EPI32_STAGE_BYTES = 8192;   // per wave: 32 rows x 64 fp32 channels

__host__ __device__ constexpr int64_t epi32_region(int64_t n) { return (n + 15) / 16 * 16; }

// the kernels that use this epilogue take only problems whose tables fit
__host__ __device__ constexpr bool epi32_tables_fit(int64_t n, bool gate) {
  return (gate ? 3 : 2) * epi32_region(n) <= EPI32_TABLE_FLOATS;
}

// The LDS tables, filled by the workgroup's NT threads in two steps: epi32_table_load issues
// every load of a thread into registers (one memory round trip, overlapped with the first chunk
// copies), epi32_table_store writes them to LDS after the kernel's first wait; a barrier must
// follow before any wave reads them. Region r < G = bias half r (0 without bias), region G =
// scale * out_scale; channels past n read 0.
template <bool GATE, int NT>
__device__ __forceinline__ void epi32_table_load(const GemmP& p, int tid, float (&v)[EPI32_TABLE_FLOATS / NT]) {
  constexpr int G = GATE ? 2 : 1;
  const int nn = (int)epi32_region(p.n);
  const int tot = (G + 1) * nn;
#pragma unroll
  for (int j = 0; j < EPI32_TABLE_FLOATS / NT; ++j) {
    const int i = tid + j * NT;
    const int r = (i >= nn) + (G == 2 && i >= 2 * nn);
    const int c = i - r * nn;
    float x = 0.f;
    if (i < tot && c < p.n) {
      if (r < G) x = p.bias ? p.bias[(int64_t)r * p.n + c] : 0.f;
      else x = (p.scale ? p.scale[c] : 1.f) * p.out_scale;
    }
    v[j] = x;
  }
}

template <bool GATE, int NT>
__device__ __forceinline__ void epi32_table_store(const GemmP& p, float* tb, int tid,
                                                  const float (&v)[EPI32_TABLE_FLOATS / NT]) {
  const int tot = ((GATE ? 2 : 1) + 1) * (int)epi32_region(p.n);
#pragma unroll
  for (int j = 0; j < EPI32_TABLE_FLOATS / NT; ++j)
    if (tid + j * NT < tot) tb[tid + j * NT] = v[j];
}

// 16-byte unit `unit` of staged row `row`, for rows of CW fp32 channels (CW / 4 units)
template <int CW>
__device__ __forceinline__ int epi32_unit(int row, int unit) { return unit ^ (row & (CW / 4 - 1)); }

// One 32-pixel block of a wave. acc0 / acc1: the two 32-row blocks (see above); q0 = the
// block's first pixel; c0 = the wave's first output channel; tb = the LDS tables.
template <bool GATE>
__device__ __forceinline__ void epi32_block(const GemmP& p, const f32x16& acc0, const f32x16& acc1, int64_t q0,
                                            int64_t c0, float* stg, const float* tb, int lane) {
  constexpr int CW = GATE ? 32 : 64;  // channels of the wave
  constexpr int G = GATE ? 2 : 1;
  const int l32 = lane & 31, hl = lane >> 5;
  const int nn = (int)epi32_region(p.n);
  // ---- 1. MFMA layout -> LDS rows
#pragma unroll
  for (int ro = 0; ro < (GATE ? 1 : 2); ++ro) {
    const int cw = ro * 32 + 16 * hl;  // first channel of this lane's run within the wave
    const int64_t run0 = c0 + cw;      // a multiple of 16: the run lies inside one table region
    const int rt = run0 < nn ? (int)run0 : 0;  // runs past n read any valid entry (not stored)
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(tb + rt + 4 * i);
      if constexpr (GATE) {
        const f32x4 b2 = *reinterpret_cast<const f32x4*>(tb + nn + rt + 4 * i);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * i + e] = (acc0[4 * i + e] + b1[e]) * (acc1[4 * i + e] + b2[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * i + e] = (ro ? acc1[4 * i + e] : acc0[4 * i + e]) + b1[e];
      }
    }
    if (p.act == ACT_GELU) {
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = gelu_erf(v[j]);
    } else if (p.act == ACT_LRELU) {
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = v[j] >= 0.f ? v[j] : v[j] * p.slope;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 sc = *reinterpret_cast<const f32x4*>(tb + G * nn + rt + 4 * i);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[4 * i + e] *= sc[e];
    }
    float* rowp = stg + l32 * CW;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<f32x4*>(rowp + 4 * epi32_unit<CW>(l32, cw / 4 + i)) =
          f32x4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
  }
  // the wave's LDS writes are complete (LDS executes a wave's instructions in order)
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  // ---- 2. row layout: LPR lanes per pixel row, 8 channels each
  constexpr int LPR = CW / 8;
  constexpr int RPR = 64 / LPR;   // rows per round
  constexpr int ROUNDS = 32 / RPR;
#pragma unroll
  for (int rd = 0; rd < ROUNDS; ++rd) {
    const int r = rd * RPR + lane / LPR;
    const int cg = (lane % LPR) * 8;
    const float* rowp = stg + r * CW;
    const f32x4 a = *reinterpret_cast<const f32x4*>(rowp + 4 * epi32_unit<CW>(r, cg / 4));
    const f32x4 b = *reinterpret_cast<const f32x4*>(rowp + 4 * epi32_unit<CW>(r, cg / 4 + 1));
    float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    const int64_t q = q0 + r;
    const int64_t ch = c0 + cg;
    if (q >= p.m || ch >= p.n) continue;
    int64_t oo, ro;
    if (p.c_mode == CM_SHUFFLE) {
      const int64_t hwi = (int64_t)p.h * p.w;
      const int64_t im = q / hwi;
      const int rr = (int)(q - im * hwi);
      const int y = rr / p.w, x = rr - (rr / p.w) * p.w;
      const int64_t cq = p.n >> 2;
      const int64_t qd = ch / cq, cc = ch - qd * cq;
      oo = ((im * 2 * p.h + 2 * y + (qd >> 1)) * 2 * p.w + 2 * x + (qd & 1)) * cq + cc;
      ro = oo;
    } else {
      oo = q * p.ldc + ch;
      ro = q * p.ldr + ch;
    }
    store_run<8>(p, v, oo, ro, ch, ch + 8 <= p.n);
  }
  // the next block's LDS writes come after these reads in program order (same wave)
  asm volatile("" ::: "memory");
}

}  // namespace clarus
