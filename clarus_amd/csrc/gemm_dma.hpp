// Multi-stage DMA-pipelined bf16 GEMM for NHWC rows without prologue (MFMA-bound shapes:
// NAFNet levels 3-4 expand and c -> c, K = 512 / 1024, K % 32 == 0), gfx950.
//
// Same math and output mapping as gemm_kernel (D[channel][pixel] = W^T . A^T on bf16 MFMA, a
// lane accumulates runs of consecutive output channels of one pixel), different data movement:
//   * a workgroup computes a 128-pixel x 128-W^T-row tile (128 output channels, or 64 with
//     SimpleGate, both halves of a channel in the same lane); its 4 waves split it 2 x 2, each
//     wave 64 pixels x 64 rows = 4 x 4 MFMA blocks per 32-k chunk;
//   * A rows and W^T rows of each 32-k chunk travel global -> LDS by direct 16-byte copies
//     (no registers) into a ring of LDS_STAGES stages, so LDS_STAGES - 1 chunks are in flight
//     while one computes; one barrier per chunk. Rows are 64 bytes, their four 16-byte units
//     XOR-swizzled by (row / 2) % 4 so the MFMA operand reads are bank-conflict free;
//   * the (tile, chunk) steps of a workgroup form one flat pipeline across tile boundaries,
//     with tiles dealt out XCD-aware (the column tiles of a pixel tile adjacent within one
//     XCD's contiguous range, so A rows come from HBM into that XCD's L2 once).
// Memory waits are explicit: a copy increments vmcnt and completes in order with the other
// copies, so waiting for chunk s is vmcnt(<copies issued after chunk s>); after an epilogue
// (its residual loads and stores share the counter) the next wait is vmcnt(0).
#pragma once

#include "gemm_lds.hpp"

namespace clarus {

constexpr int DMA_P = 128;       // pixels per tile
constexpr int DMA_R = 128;       // W^T rows per tile
constexpr int DMA_KC = 32;       // k per chunk
constexpr int DMA_STAGES = 4;    // LDS ring depth
constexpr int DMA_ROWB = 64;     // bytes per staged row (32 bf16)
constexpr int DMA_ABYTES = DMA_P * DMA_ROWB;   // 8 KiB
constexpr int DMA_WBYTES = DMA_R * DMA_ROWB;   // 8 KiB
constexpr int DMA_STAGE = DMA_ABYTES + DMA_WBYTES;
constexpr int DMA_COPIES = DMA_STAGE / 1024 / 4;  // 16-byte copies per lane (one per 1 KiB per wave) per stage
__host__ __device__ constexpr int dma_lds_bytes() { return DMA_STAGES * DMA_STAGE; }

__device__ __forceinline__ int dma_swz(int row, int unit) { return unit ^ ((row >> 1) & 3); }

__device__ __forceinline__ void wait_vm(int n) {
  // vmcnt(n) for n in {0, DMA_COPIES, 2 DMA_COPIES} (expcnt / lgkmcnt untouched)
  if (n == 0) __builtin_amdgcn_s_waitcnt(0x0F70);
  else if (n == DMA_COPIES) __builtin_amdgcn_s_waitcnt(0x0F70 | DMA_COPIES);
  else __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * DMA_COPIES));
}

template <bool GATE>
__global__ void __launch_bounds__(256) gemm_dma_kernel(const GemmP p) {
  static_assert(DMA_COPIES == 4 && 2 * DMA_COPIES < 16, "wait encoding");
  constexpr int G = GATE ? 2 : 1;
  constexpr int TNO = DMA_R / G;  // output channels per tile
  constexpr int WCH = TNO / 2;    // output channels per wave
  constexpr int RUN = WCH / 4;    // contiguous channels per lane (16, gate 8)
  extern __shared__ __attribute__((aligned(16))) unsigned char ring[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lc = lane & 15, lg = lane >> 4;
  const int wp = wave & 1, wn = wave >> 1;
  const int64_t K = p.k;
  const int nch = (int)(K / DMA_KC);
  const int ntn = (int)cdiv(p.n, TNO);
  const int T = (int)p.ptiles * ntn;  // the host checks that this fits 31 bits
  const unsigned char* A = (const unsigned char*)p.a;
  const unsigned char* Wt = (const unsigned char*)p.wt;

  const int xcd = blockIdx.x & 7;
  const int per = gridDim.x >> 3;
  const int span = (T + 7) >> 3;
  const int t0 = xcd * span + (blockIdx.x >> 3);
  const int t_end = (xcd + 1) * span < T ? (xcd + 1) * span : T;
  const int ntiles = t0 < t_end ? (t_end - t0 + per - 1) / per : 0;
  const int nsteps = ntiles * nch;

  // copies of one chunk into ring stage st: 16 KiB = 16 x 1 KiB; wave w takes the KiBs w, w + 4,
  // w + 8, w + 12 (the first 8 are A, the rest W^T). A KiB is 16 rows x 64 B: lane i fills
  // row 16 j + i / 4, slot i % 4 with source unit dma_swz(row, slot). The issue position
  // (tile, chunk) advances incrementally (no divisions per step).
  int is_tile = 0, is_chunk = 0, is_stage = 0;
  const unsigned char* src_base[DMA_COPIES];  // this lane's source at k = 0 for the issue tile
  auto set_issue_tile = [&]() __attribute__((always_inline)) {
    const int t = t0 + is_tile * per;
    const int pt = t / ntn;
    const int nt = t - pt * ntn;
#pragma unroll
    for (int j = 0; j < DMA_COPIES; ++j) {
      const int kib = wave + 4 * j;
      const int row = (kib & 7) * 16 + (lane >> 2);
      const int unit = dma_swz(row, lane & 3);
      if (kib < 8) {
        int64_t q = (int64_t)pt * DMA_P + row;
        if (q > p.m - 1) q = p.m - 1;  // rows past M: any valid row, its outputs are not stored
        src_base[j] = A + (q * p.lda + unit * 8) * 2;
      } else {
        int half, ch;
        if constexpr (GATE) {
          half = row >> 6;
          const int rl = row & 63, w2 = rl >> 5, r2 = rl & 31;
          ch = w2 * 32 + ((r2 & 15) >> 2) * 8 + (r2 >> 4) * 4 + (r2 & 3);
        } else {
          half = 0;
          const int w2 = row >> 6, r2 = row & 63;
          ch = w2 * 64 + ((r2 & 15) >> 2) * 16 + (r2 >> 4) * 4 + (r2 & 3);
        }
        int64_t c = (int64_t)nt * TNO + ch;
        if (c > p.n - 1) c = p.n - 1;  // channels past N: not stored
        src_base[j] = Wt + ((half * p.n + c) * K + unit * 8) * 2;
      }
    }
  };
  auto issue = [&]() __attribute__((always_inline)) {
    const int64_t kb = (int64_t)is_chunk * (DMA_KC * 2);
    unsigned char* st = ring + is_stage * DMA_STAGE;
#pragma unroll
    for (int j = 0; j < DMA_COPIES; ++j)
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src_base[j] + kb),
                                       (__attribute__((address_space(3))) void*)(st + (wave + 4 * j) * 1024), 16, 0,
                                       0);
    is_stage = (is_stage + 1) & (DMA_STAGES - 1);
    if (++is_chunk == nch) {
      is_chunk = 0;
      ++is_tile;
      set_issue_tile();
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto wrow = [&](int rb) { return GATE ? ((rb >> 1) * 64 + wn * 32 + (rb & 1) * 16) : (wn * 64 + rb * 16); };

  set_issue_tile();
  for (int s = 0; s < DMA_STAGES - 1; ++s)
    if (s < nsteps) issue();
  int s = 0;        // global step (chunk) index
  int c_stage = 0;  // ring stage of step s

  for (int tl = 0; tl < ntiles; ++tl) {
    // ---- the tile's K loop: one chunk per step
    for (int kc = 0; kc < nch; ++kc, ++s) {
      // chunk s landed (this thread's copies), then everyone's; stage (s - 1) % STAGES is free.
      // At a tile's first chunk the previous epilogue's memory ops share the counter: wait for all.
      const int later = (nsteps - 1 - s) < (DMA_STAGES - 2) ? (nsteps - 1 - s) : (DMA_STAGES - 2);
      wait_vm(kc == 0 ? 0 : later * DMA_COPIES);
      barrier_keep_vm();
      if (s + DMA_STAGES - 1 < nsteps) issue();
      const unsigned char* st = ring + c_stage * DMA_STAGE;
      const unsigned char* wb = st + DMA_ABYTES;
      bf16x8 wf[4];
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        const int r = wrow(rb) + lc;
        wf[rb] = *reinterpret_cast<const bf16x8*>(wb + r * DMA_ROWB + dma_swz(r, lg) * 16);
      }
#pragma unroll
      for (int pb = 0; pb < 4; ++pb) {
        const int r = wp * 64 + pb * 16 + lc;
        const bf16x8 af = *reinterpret_cast<const bf16x8*>(st + r * DMA_ROWB + dma_swz(r, lg) * 16);
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) acc[pb][rb] = mfma_bf16(wf[rb], af, acc[pb][rb]);
      }
      c_stage = (c_stage + 1) & (DMA_STAGES - 1);
    }

    // ---- epilogue of the tile
    {
      const int t = t0 + tl * per;
      const int pt = t / ntn, nt = t - pt * ntn;
      const int e0 = wn * WCH + lg * RUN;
      const int64_t run0 = (int64_t)nt * TNO + e0;
      const bool full_n = run0 + RUN <= p.n;
      // the run's bias (both gate halves) and scale * out_scale, straight from global memory
      float b1[RUN], b2[GATE ? RUN : 1], sc[RUN];
#pragma unroll
      for (int i = 0; i < RUN; ++i) {
        const bool ok = run0 + i < p.n;
        b1[i] = (p.bias && ok) ? p.bias[run0 + i] : 0.f;
        if constexpr (GATE) b2[i] = (p.bias && ok) ? p.bias[p.n + run0 + i] : 0.f;
        sc[i] = ((p.scale && ok) ? p.scale[run0 + i] : 1.f) * p.out_scale;
      }
#pragma unroll
      for (int pb = 0; pb < 4; ++pb) {
        const int64_t q = (int64_t)pt * DMA_P + wp * 64 + pb * 16 + lc;
        float v[RUN];
        if constexpr (GATE) {
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              v[j * 4 + i] = (acc[pb][j][i] + b1[j * 4 + i]) * (acc[pb][2 + j][i] + b2[j * 4 + i]);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) v[j * 4 + i] = acc[pb][j][i] + b1[j * 4 + i];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[pb][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (q >= p.m) continue;
        if (p.act == ACT_GELU) {
#pragma unroll
          for (int i = 0; i < RUN; ++i) v[i] = gelu_erf(v[i]);
        } else if (p.act == ACT_LRELU) {
#pragma unroll
          for (int i = 0; i < RUN; ++i) v[i] = v[i] >= 0.f ? v[i] : v[i] * p.slope;
        }
#pragma unroll
        for (int i = 0; i < RUN; ++i) v[i] *= sc[i];
        int64_t oo, ro;
        if (p.c_mode == CM_SHUFFLE) {
          const int64_t hwi = (int64_t)p.h * p.w;
          const int64_t im = q / hwi;
          const int rr = (int)(q - im * hwi);
          const int y = rr / p.w, x = rr - (rr / p.w) * p.w;
          const int64_t cq = p.n >> 2;
          const int64_t qd = run0 / cq, cc = run0 - qd * cq;
          oo = ((im * 2 * p.h + 2 * y + (qd >> 1)) * 2 * p.w + 2 * x + (qd & 1)) * cq + cc;
          ro = oo;
        } else {
          oo = q * p.ldc + run0;
          ro = q * p.ldr + run0;
        }
        store_run<RUN>(p, v, oo, ro, run0, full_n);
      }
    }
  }
}

}  // namespace clarus
