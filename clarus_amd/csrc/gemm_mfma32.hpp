// DMA-pipelined bf16 GEMM on 32x32x16 MFMAs with 64-k chunks (MFMA-bound NHWC shapes without
// prologue: NAFNet levels 2-4 expand and c -> c, K % 64 == 0), gfx950.
//
// Same math and output mapping as gemm_kernel (D[channel][pixel] = W^T . A^T on bf16 MFMA, a
// lane accumulates a run of consecutive output channels of one pixel). Three measured facts set
// the shape of this kernel:
//   * a global -> LDS copy instruction moves 64 x 16 B; when those bytes are 64-byte pieces of
//     16 rows, L2 delivers 9-17 TB/s, when they are 128-byte pieces of 8 rows it delivers
//     ~33 TB/s. A chunk is therefore 64 k (128 bytes of every row);
//   * 32x32x16 bf16 MFMAs issued back to back by one wave per SIMD reach ~2.3 PFLOP/s, the
//     16x16x32 ones ~1.3 (they need two waves per SIMD);
//   * on the NAFNet shapes two workgroups per CU with a 2-stage ring (64 KiB each) beat one
//     workgroup with a 3- or 4-stage ring: a single wave per SIMD serializes copy issue, LDS
//     reads and MFMAs, where two interleave them;
//   * LDS reads run at ~128 B/clk per CU: a wave computes 64 pixels x 64 rows (2 x 2 MFMA
//     blocks) from 4 fragment reads per 16-k step.
// Data movement:
//   * a workgroup computes a 128-pixel x 128-W^T-row tile (128 output channels, or 64 with
//     SimpleGate, both halves of a channel in the same lane); its 4 waves split it 2 x 2;
//   * A rows and W^T rows of each 64-k chunk travel global -> LDS by direct 16-byte copies into
//     a ring of M32_STAGES stages of 32 KiB; rows are 128 bytes, their eight 16-byte units
//     XOR-swizzled by (row / 2) % 8 so the fragment reads of 16 consecutive rows hit 16
//     distinct 16-byte bank groups;
//   * the (tile, chunk) steps of a workgroup form one flat pipeline across tile boundaries;
//     tiles are dealt out XCD-aware (a contiguous tile range per XCD, the column tiles of a
//     pixel tile adjacent).
// Output mapping of the 32x32x16 MFMA: lane l holds D[8 (j / 4) + 4 (l / 32) + j % 4][l % 32]
// in accumulator element j. W^T rows are permuted when staged so that element j of lane l is
// channel 16 (l / 32) + j of its 32-row block: every lane owns 16 consecutive channels.
// Memory waits are explicit: with two stages the chunk waited for is always the newest copy
// group, so every wait is vmcnt(0) (it also covers an epilogue's loads and stores).
// Space-to-depth rows (p.s2d, the 2x2 stride-2 down conv): A row q is the window of output
// pixel q, k = (2 dy + dx) cin + c. Its first 2 cin elements are input row 2y at pixels 2x, 2x + 1
// and its last 2 cin are input row 2y + 1 at the same pixels, each contiguous: a lane's copy
// source starts at (2y, 2x) and jumps by (w - 2) cin elements once k reaches 2 cin (a chunk
// boundary, since cin % 32 == 0).
#pragma once

#include "gemm_epi32.hpp"

namespace clarus {

constexpr int M32_P = 128;                        // pixels per tile
constexpr int M32_R = 128;                        // W^T rows per tile
constexpr int M32_KC = 64;                        // k per chunk
constexpr int M32_ROWB = 128;                     // bytes per staged row (64 bf16)
constexpr int M32_ABYTES = M32_P * M32_ROWB;      // 16 KiB
constexpr int M32_WBYTES = M32_R * M32_ROWB;      // 16 KiB
constexpr int M32_STAGE = M32_ABYTES + M32_WBYTES;
constexpr int M32_COPIES = M32_STAGE / 1024 / 4;  // 16-byte copies per lane per stage (8)
constexpr int M32_RUN = 16;                       // consecutive output channels per lane
constexpr int M32_STAGES = 2;                     // LDS ring depth
constexpr int M32_RING = M32_STAGES * M32_STAGE;  // 64 KiB
constexpr int M32_LDS = M32_RING + EPI32_TABLE_FLOATS * 4;  // + epilogue tables: 80 KiB, two workgroups per CU
static_assert(M32_ABYTES / 1024 == 4 * 4, "copies j < 4 of a lane are the A KiBs (4 waves)");

__device__ __forceinline__ int m32_swz(int row, int unit) { return unit ^ ((row >> 1) & 7); }

__device__ __forceinline__ f32x16 mfma32_bf16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}


// two workgroups per CU: registers capped at 256 per lane
template <bool GATE>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) gemm_mfma32_kernel(const GemmP p) {
  constexpr int STAGES = M32_STAGES;
  static_assert(STAGES == 2, "the waits below assume one chunk in flight behind the computed one");
  constexpr int TNO = GATE ? M32_R / 2 : M32_R;  // output channels per tile
  extern __shared__ __attribute__((aligned(16))) unsigned char ring[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hl = lane >> 5;
  const int wp = wave & 1, wn = wave >> 1;
  const int64_t K = p.k;
  const int nch = (int)(K / M32_KC);
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
  if (nsteps == 0) return;  // nothing to do (before any LDS or memory traffic)

  // epilogue tables (bias, scale) in LDS (the host checks that they fit)
  float* tb = reinterpret_cast<float*>(ring + M32_RING);

  // copies of one chunk into ring stage st: 32 KiB = 32 x 1 KiB; wave w takes the KiBs w + 4 j
  // (the first 16 are A, the rest W^T). A KiB is 8 rows x 128 B: lane i fills row 8 (KiB % 16)
  // + i / 8, slot i % 8 with source unit m32_swz(row, slot). The issue position (tile, chunk)
  // advances incrementally.
  int is_tile = 0, is_chunk = 0, is_stage = 0;
  const unsigned char* src_base[M32_COPIES];  // this lane's source at k = 0 for the issue tile
  auto set_issue_tile = [&]() __attribute__((always_inline)) {
    const int t = t0 + is_tile * per;
    const int pt = t / ntn;
    const int nt = t - pt * ntn;
#pragma unroll
    for (int j = 0; j < M32_COPIES; ++j) {
      const int kib = wave + 4 * j;
      const int row = (kib & 15) * 8 + (lane >> 3);
      const int unit = m32_swz(row, lane & 7);
      if (kib < 16) {
        int64_t q = (int64_t)pt * M32_P + row;
        if (q > p.m - 1) q = p.m - 1;  // rows past M: any valid row, its outputs are not stored
        if (p.s2d) {
          const int wo = p.w >> 1, hwo = (p.h >> 1) * wo;
          const int64_t img = q / hwo;
          const int r = (int)(q - img * hwo);
          const int py = r / wo, px = r - py * wo;
          src_base[j] = A + ((((img * p.h + 2 * py) * p.w + 2 * px) * p.cin) + unit * 8) * 2;
        } else {
          src_base[j] = A + (q * p.lda + unit * 8) * 2;
        }
      } else {
        // W^T row `row` = wave-row wr, block rb, block row rr = 8 g + 4 h + i holds channel
        // 16 h + 4 g + i of its 32-channel run (gate: block rb is the SimpleGate half)
        const int wr = row >> 6, rb = (row >> 5) & 1, rr = row & 31;
        const int cw = 16 * ((rr >> 2) & 1) + 4 * (rr >> 3) + (rr & 3);
        const int half = GATE ? rb : 0;
        const int ch = GATE ? wr * 32 + cw : wr * 64 + rb * 32 + cw;
        int64_t c = (int64_t)nt * TNO + ch;
        if (c > p.n - 1) c = p.n - 1;  // channels past N: not stored
        src_base[j] = Wt + ((half * p.n + c) * K + unit * 8) * 2;
      }
    }
  };
  // space-to-depth: the A source jumps to input row 2y + 1 from chunk s2d_kc on
  const int s2d_kc = p.s2d ? (2 * p.cin) / M32_KC : nch;
  const int64_t s2d_jump = p.s2d ? (int64_t)(p.w - 2) * p.cin * 2 : 0;
  auto issue = [&]() __attribute__((always_inline)) {
    const int kb = is_chunk * (M32_KC * 2);
    const int64_t ka = kb + (is_chunk >= s2d_kc ? s2d_jump : 0);  // A copies (j < 4: KiBs 0-15)
    unsigned char* st = ring + is_stage * M32_STAGE;
#pragma unroll
    for (int j = 0; j < M32_COPIES; ++j)
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src_base[j] + (j < 4 ? ka : kb)),
                                       (__attribute__((address_space(3))) void*)(st + (wave + 4 * j) * 1024), 16, 0,
                                       0);
    is_stage = is_stage + 1 == STAGES ? 0 : is_stage + 1;
    if (++is_chunk == nch) {
      is_chunk = 0;
      ++is_tile;
      set_issue_tile();
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.f;

  // MFMA fragments of one 16-k step, double-buffered: step ks + 1 is read while step ks computes
  bf16x8 wf[2][2], af[2][2];
  auto load_frags = [&](int buf, int stage, int ks) __attribute__((always_inline)) {
    const unsigned char* st = ring + stage * M32_STAGE;
    const int u = 2 * ks + hl;  // 16-byte unit: k = 16 ks + 8 (l / 32) .. + 8
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int r = wn * 64 + rb * 32 + l32;
      wf[buf][rb] = *reinterpret_cast<const bf16x8*>(st + M32_ABYTES + r * M32_ROWB + m32_swz(r, u) * 16);
    }
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
      const int r = wp * 64 + pb * 32 + l32;
      af[buf][pb] = *reinterpret_cast<const bf16x8*>(st + r * M32_ROWB + m32_swz(r, u) * 16);
    }
  };
  auto products = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) acc[pb][rb] = mfma32_bf16(wf[buf][rb], af[buf][pb], acc[pb][rb]);
  };

  set_issue_tile();
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < nsteps) issue();
  // the tables' loads overlap the first chunk copies; they are stored after the first wait and
  // published by the barrier that ends chunk 0
  float tv[EPI32_TABLE_FLOATS / 256];
  epi32_table_load<GATE, 256>(p, tid, tv);
  // chunk 0 landed everywhere; the ring's last stage is free
  wait_vmcnt<0>();
  barrier_keep_vm();
  if (STAGES - 1 < nsteps) issue();
  epi32_table_store<GATE, 256>(p, tb, tid, tv);
  load_frags(0, 0, 0);
  int s = 0;        // global step (chunk) index
  int c_stage = 0;  // ring stage of step s

  for (int tl = 0; tl < ntiles; ++tl) {
    // ---- the tile's K loop: one 64-k chunk per step, 4 MFMA steps of 16 k
    int last_stage = 0;     // ring stage of the tile's last chunk: the epilogue's staging area
    bool deferred = false;  // the copy that would refill that stage waits for the epilogue
    for (int kc = 0; kc < nch; ++kc, ++s) {
#pragma unroll
      for (int ks = 0; ks < M32_KC / 16 - 1; ++ks) {
        load_frags((ks + 1) & 1, c_stage, ks + 1);
        products(ks & 1);
      }
      // last MFMA step: chunk s + 1 must have landed (this thread's copies, then everyone's);
      // with two stages it is the newest copy group, so the wait is for all. After the barrier
      // every wave has finished its LDS reads of chunk s, whose stage takes chunk s + 2 (after
      // the epilogue when chunk s ends a tile).
      const int n_stage = c_stage + 1 == STAGES ? 0 : c_stage + 1;
      if (s + 1 < nsteps) {
        wait_vmcnt<0>();
        barrier_keep_vm();
        if (s + STAGES < nsteps) {
          if (kc == nch - 1) deferred = true;
          else issue();
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
    // wp * 64 + [0, 64) and channels wn * 64 (gate: wn * 32) + [0, 64 (32))
    {
      const int t = t0 + tl * per;
      const int pt = t / ntn, nt = t - pt * ntn;
      float* stg = reinterpret_cast<float*>(ring + last_stage * M32_STAGE + wave * EPI32_STAGE_BYTES);
      const int64_t c0 = (int64_t)nt * TNO + (GATE ? wn * 32 : wn * 64);
#pragma unroll
      for (int pb = 0; pb < 2; ++pb)
        epi32_block<GATE>(p, acc[pb][0], acc[pb][1], (int64_t)pt * M32_P + wp * 64 + pb * 32, c0, stg, tb, lane);
      if (deferred) {  // every wave is done with its staging rows: refill the stage
        barrier_keep_vm();
        issue();
      }
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.f;
    }
  }
}

}  // namespace clarus
