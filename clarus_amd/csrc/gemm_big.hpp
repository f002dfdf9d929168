// Big-tile DMA-pipelined bf16 GEMM on 32x32x16 MFMAs (long-K NHWC shapes without prologue,
// K % 64 == 0), gfx950.
//
// Same math, operand staging and output mapping as gemm_mfma32_kernel (D[channel][pixel] =
// W^T . A^T, 64-k chunks copied global -> LDS by direct 16-byte copies into a swizzled ring,
// every lane owning 16 consecutive output channels of one pixel), with a larger tile:
//   * a workgroup computes 128 * WP pixels x 256 W^T rows (256 output channels, or 128 with
//     SimpleGate); its 4 * WP waves each compute 128 pixels x 64 rows (4 x 2 MFMA blocks);
//   * WP = 2: 8 waves (two per SIMD), a 2-stage ring of 64 KiB stages (128 KiB, one workgroup
//     per CU); WP = 1: 4 waves, a 3-stage ring of 48 KiB stages (144 KiB).
// Why: LDS serves both the fragment reads and the global -> LDS copies, at ~105 B/clk per CU
// together (measured). A 64 x 64 wave tile in a 128 x 128 workgroup tile moves 6 KiB through
// LDS per 131 kflop; a 128 x 64 wave tile in a 256 x 256 workgroup tile moves 8 KiB per
// 262 kflop, and every chunk copied from L2 feeds twice the products. Inner-loop benchmark
// (LDS reads + copies + MFMAs, no HBM): 1.33 vs 1.57 PFLOP/s.
// Memory waits are explicit vmcnt counts: at the wait for chunk s + 1 the copy groups of chunks
// s + 2 .. s + STAGES - 1 may stay in flight. After a tile's epilogue (its residual loads and
// output stores also count in vmcnt) the next wait drains everything once. The epilogue runs
// through LDS rows (gemm_epi32.hpp) staged in the ring stage of the tile's last chunk; the copy
// that would refill that stage is issued after the epilogue.
#pragma once

#include "gemm_mfma32.hpp"

namespace clarus {

constexpr int BIG_R = 256;        // W^T rows per tile
constexpr int BIG_KC = 64;        // k per chunk
constexpr int BIG_ROWB = 128;     // bytes per staged row
constexpr int BIG_RUN = 16;       // consecutive output channels per lane

template <int WP>
struct BigCfg {
  static constexpr int P = 128 * WP;                       // pixels per tile
  static constexpr int NW = 4 * WP;                        // waves
  static constexpr int NT = 64 * NW;                       // threads
  static constexpr int ABYTES = P * BIG_ROWB;
  static constexpr int STAGE = ABYTES + BIG_R * BIG_ROWB;  // 64 KiB (WP 2) / 48 KiB (WP 1)
  static constexpr int STAGES = WP == 2 ? 2 : 3;
  static constexpr int RING = STAGES * STAGE;              // 128 / 144 KiB
  static constexpr int LDS = RING + EPI32_TABLE_FLOATS * 4;  // + epilogue tables
  static constexpr int COPIES = STAGE / 1024 / NW;         // 16-byte copies per lane per stage
  static constexpr int AKIB = ABYTES / 1024;               // KiBs of A per stage
};

template <int N>
__device__ __forceinline__ void wait_groups(int groups) {
  // vmcnt(groups * N) for groups in {0, 1}: the copy groups newer than the awaited chunk
  if (groups <= 0) wait_vmcnt<0>();
  else wait_vmcnt<N>();
}

template <bool GATE, int WP>
__global__ void __launch_bounds__(64 * 4 * WP) __attribute__((amdgpu_waves_per_eu(WP, WP)))
gemm_big_kernel(const GemmP p) {
  using C = BigCfg<WP>;
  constexpr int STAGES = C::STAGES;
  static_assert(STAGES == 2 || STAGES == 3, "the waits below allow at most one newer copy group");
  constexpr int TNO = GATE ? BIG_R / 2 : BIG_R;  // output channels per tile
  extern __shared__ __attribute__((aligned(16))) unsigned char ring[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hl = lane >> 5;
  const int wp = wave % WP, wn = wave / WP;  // pixel group (128 px), row group (64 rows)
  const int64_t K = p.k;
  const int nch = (int)(K / BIG_KC);
  const int ntn = (int)cdiv(p.n, TNO);
  const int T = (int)p.ptiles * ntn;  // the host checks that this fits 31 bits
  const unsigned char* A = (const unsigned char*)p.a;
  const unsigned char* Wt = (const unsigned char*)p.wt;

  // XCD-aware deal: a contiguous tile range per XCD (blockIdx % 8), the column tiles of a pixel
  // tile adjacent, so an XCD's L2 holds the A rows and W^T rows its workgroups share
  const int xcd = blockIdx.x & 7;
  const int per = gridDim.x >> 3;
  const int span = (T + 7) >> 3;
  const int t0 = xcd * span + (blockIdx.x >> 3);
  const int t_end = (xcd + 1) * span < T ? (xcd + 1) * span : T;
  const int ntiles = t0 < t_end ? (t_end - t0 + per - 1) / per : 0;
  const int nsteps = ntiles * nch;
  if (nsteps == 0) return;  // nothing to do (before any LDS or memory traffic)

  // epilogue tables (bias, scale) in LDS (the host checks that they fit)
  float* tb = reinterpret_cast<float*>(ring + C::RING);

  // copies of one chunk into a stage: KiB j of the stage is 8 rows x 128 B (A rows first, then
  // W^T rows); wave w takes the KiBs w + NW * i. Lane l fills row 8 (KiB) + l / 8, slot l % 8,
  // from source unit m32_swz(row, slot). Sources are 32-bit byte offsets from the issue tile's
  // A and W^T bases (wave-uniform), so a copy costs one VGPR.
  int is_tile = 0, is_chunk = 0, is_stage = 0;
  const unsigned char* a_tile = A;
  const unsigned char* w_tile = Wt;
  uint32_t src_off[C::COPIES];
  auto set_issue_tile = [&]() __attribute__((always_inline)) {
    const int t = t0 + is_tile * per;
    const int pt = t / ntn;
    const int nt = t - pt * ntn;
    a_tile = A + (int64_t)pt * C::P * p.lda * 2;
    w_tile = Wt + (int64_t)nt * TNO * K * 2;
    const int64_t rows_left = p.m - 1 - (int64_t)pt * C::P;  // last valid row of the tile
    const int64_t ch_left = p.n - 1 - (int64_t)nt * TNO;      // last valid channel of the tile
#pragma unroll
    for (int j = 0; j < C::COPIES; ++j) {
      const int kib = wave + C::NW * j;
      const int unit = (lane & 7);
      if (kib < C::AKIB) {
        const int row = kib * 8 + (lane >> 3);
        // rows past M read the tile's last valid row; their outputs are not stored
        const int64_t q = row < rows_left ? row : rows_left;
        src_off[j] = (uint32_t)((q * p.lda + m32_swz(row, unit) * 8) * 2);
      } else {
        // W^T row `row`: row group wr = row / 64, block rb, block row rr = 8 g + 4 h + i holds
        // channel 16 h + 4 g + i of its 32-channel run (gate: block rb is the SimpleGate half)
        const int row = (kib - C::AKIB) * 8 + (lane >> 3);
        const int wr = row >> 6, rb = (row >> 5) & 1, rr = row & 31;
        const int cw = 16 * ((rr >> 2) & 1) + 4 * (rr >> 3) + (rr & 3);
        const int half = GATE ? rb : 0;
        const int ch = GATE ? wr * 32 + cw : wr * 64 + rb * 32 + cw;
        const int64_t c = ch < ch_left ? ch : ch_left;  // channels past N: not stored
        src_off[j] = (uint32_t)(((half * p.n + c) * K + m32_swz(row, unit) * 8) * 2);
      }
    }
  };
  auto issue = [&]() __attribute__((always_inline)) {
    const int kb = is_chunk * (BIG_KC * 2);
    unsigned char* st = ring + is_stage * C::STAGE;
#pragma unroll
    for (int j = 0; j < C::COPIES; ++j) {
      const unsigned char* src = ((wave + C::NW * j) < C::AKIB ? a_tile : w_tile) + src_off[j] + kb;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                       (__attribute__((address_space(3))) void*)(st + (wave + C::NW * j) * 1024), 16,
                                       0, 0);
    }
    is_stage = is_stage + 1 == STAGES ? 0 : is_stage + 1;
    if (++is_chunk == nch) {
      is_chunk = 0;
      ++is_tile;
      set_issue_tile();
    }
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.f;

  // MFMA fragments of one 16-k step, double-buffered: step ks + 1 is read while step ks computes.
  // The swizzle term of every fragment row r = 32 b + l % 32 is ((l % 32) / 2) % 8, so one
  // address per operand and k-step serves all blocks (block offsets are immediates).
  bf16x8 wf[2][2], af[2][4];
  const int g = (l32 >> 1) & 7;
  const int row_a = (wp * 128 + l32) * BIG_ROWB;
  const int row_w = C::ABYTES + (wn * 64 + l32) * BIG_ROWB;
  auto load_frags = [&](int buf, int stage, int ks) __attribute__((always_inline)) {
    const unsigned char* st = ring + stage * C::STAGE + (((2 * ks + hl) ^ g) << 4);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
      wf[buf][rb] = *reinterpret_cast<const bf16x8*>(st + row_w + rb * 32 * BIG_ROWB);
#pragma unroll
    for (int pb = 0; pb < 4; ++pb)
      af[buf][pb] = *reinterpret_cast<const bf16x8*>(st + row_a + pb * 32 * BIG_ROWB);
  };
  auto products = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int pb = 0; pb < 4; ++pb)
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) acc[pb][rb] = mfma32_bf16(wf[buf][rb], af[buf][pb], acc[pb][rb]);
  };

  set_issue_tile();
  int issued = 0;
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < nsteps) { issue(); ++issued; }
  // the tables' loads overlap the first chunk copies; they are stored after the first wait and
  // published by the barrier that ends chunk 0
  float tv[EPI32_TABLE_FLOATS / C::NT];
  epi32_table_load<GATE, C::NT>(p, tid, tv);
  // chunk 0 landed everywhere (newer groups may stay in flight)
  wait_groups<C::COPIES>(issued - 1);
  barrier_keep_vm();
  if (issued < nsteps) { issue(); ++issued; }
  epi32_table_store<GATE, C::NT>(p, tb, tid, tv);
  load_frags(0, 0, 0);
  int s = 0;        // global step (chunk) index
  int c_stage = 0;  // ring stage of step s
  bool drained = false;  // an epilogue ran since the last wait: drain all

  for (int tl = 0; tl < ntiles; ++tl) {
    // ---- the tile's K loop: one 64-k chunk per step, 4 MFMA steps of 16 k
    int last_stage = 0;     // ring stage of the tile's last chunk: the epilogue's staging area
    bool deferred = false;  // the copy that would refill that stage waits for the epilogue
    for (int kc = 0; kc < nch; ++kc, ++s) {
#pragma unroll
      for (int ks = 0; ks < BIG_KC / 16 - 1; ++ks) {
        load_frags((ks + 1) & 1, c_stage, ks + 1);
        products(ks & 1);
      }
      // last MFMA step: chunk s + 1 must have landed (this thread's copies, then everyone's).
      // Issued so far: chunks < `issued`; the ones after s + 1 may stay in flight. After the
      // barrier every wave has finished its LDS reads of chunk s, whose stage takes the next
      // chunk (after the epilogue when chunk s ends a tile).
      const int n_stage = c_stage + 1 == STAGES ? 0 : c_stage + 1;
      if (s + 1 < nsteps) {
        if (drained) wait_vmcnt<0>();
        else wait_groups<C::COPIES>(issued - (s + 2));
        drained = false;
        barrier_keep_vm();
        if (issued < nsteps) {
          if (kc == nch - 1) deferred = true;
          else { issue(); ++issued; }
        }
        load_frags(0, n_stage, 0);
      } else {
        barrier_keep_vm();  // the last chunk: every wave is past its reads of this stage
      }
      last_stage = c_stage;
      products(1);
      c_stage = n_stage;
    }

    // ---- epilogue of the tile through LDS rows (gemm_epi32.hpp): wave (wp, wn) owns pixels
    // wp * 128 + [0, 128) and channels wn * 64 (gate: wn * 32) + [0, 64 (32))
    {
      const int t = t0 + tl * per;
      const int pt = t / ntn, nt = t - pt * ntn;
      float* stg = reinterpret_cast<float*>(ring + last_stage * C::STAGE + wave * EPI32_STAGE_BYTES);
      const int64_t c0 = (int64_t)nt * TNO + (GATE ? wn * 32 : wn * 64);
#pragma unroll
      for (int pb = 0; pb < 4; ++pb)
        epi32_block<GATE>(p, acc[pb][0], acc[pb][1], (int64_t)pt * C::P + wp * 128 + pb * 32, c0, stg, tb, lane);
      if (deferred) {  // every wave is done with its staging rows: refill the stage
        barrier_keep_vm();
        issue();
        ++issued;
      }
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.f;
      drained = true;
    }
  }
}

}  // namespace clarus
