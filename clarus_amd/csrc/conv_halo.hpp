// 3x3 convolution (stride 1, zero padding 1, optional nearest-x2 input) on output tiles with an
// LDS halo, gfx950. bf16 input and weights, fp32 accumulation.
//
// The implicit-GEMM formulation reads every input pixel nine times (once per tap); here a
// workgroup instead
//   * keeps the weights of its TR output channels resident in LDS for the whole kernel
//     (W^T [TR][9 cin], rows padded by 16 bytes so the MFMA operand reads are conflict free),
//   * walks 8 x 32-pixel output tiles (16 x 32 with the x2 upsample); per 32-input-channel chunk,
//     the tile's input halo ((8 + 2) x (32 + 2) pixels, or 10 x 18 at input resolution with the x2
//     upsample) arrives by
//     direct global->LDS copies into a ring of STAGES buffers; taps outside the image read a
//     zero page, so the padding costs no branches,
//   * and computes all nine taps from the halo: each of the 8 waves owns RW output rows (2 blocks
//     of 16 pixels each) and all TR channels, one bf16 MFMA (16 x 16 x 32) per (tap, row, pixel
//     block, 16 channels); two waves per SIMD hide each other's LDS latency. The weight fragments
//     of a tap are read from LDS once per wave for all its rows: with one row per wave the
//     x2-upsample conv's K loop was bound by those reads (8 waves x 9 taps x 6 KiB per chunk;
//     a timing variant reading a quarter of them ran the loop 30 % faster), hence RW = 2 there.
// The K loop of a tile is one chunk per step with a single barrier; the epilogue (bias,
// LeakyReLU, out_scale, residual, 16-byte stores into a channel slice of the output) runs once
// per tile outside it, and the next tile's first halo is already in flight by then. The bias
// comes from an LDS table, and a tile's residual loads and stores are issued only after the next
// tile's first chunk has been waited for: loads and copies complete in issue order, so a global
// load in the epilogue waited for every halo copy in flight, and the stores were waited for with
// the next tile's first copies (2 - 2.5 us per tile at a tile boundary). NCHW fp32
// output (c_mode NCHW, the NAFNet ending conv with its global residual) is stored per channel
// plane; TR = 16 serves narrow outputs (cout <= 16, e.g. 3 image channels).
#pragma once

#include "gemm_lds.hpp"

namespace clarus {

constexpr int CH_TW = 32;  // output tile columns
constexpr int CH_KC = 32;  // input channels per chunk

// output rows per wave: 2 with the x2 upsample (16-row tiles), else 1 (8-row tiles)
__host__ __device__ constexpr int conv_halo_rw(bool up2) { return up2 ? 2 : 1; }

template <bool UP2>
struct HaloGeom {
  static constexpr int th = 8 * conv_halo_rw(UP2);                   // output tile rows: 16 / 8
  static constexpr int rows = UP2 ? th / 2 + 2 : th + 2;            // 10 / 10
  static constexpr int cols = UP2 ? CH_TW / 2 + 2 : CH_TW + 2;      // 18 / 34
  static constexpr int px = rows * cols;                            // 180 / 340
  static constexpr int px_pad = (px + 127) / 128 * 128;             // a whole number of 16-pixel copies per wave
  static constexpr int bytes = px_pad * 64;                         // 32 bf16 channels per pixel
  static constexpr int copies = px_pad / 128;                       // 16-byte copies per lane per stage (8 waves)
};
static_assert(HaloGeom<true>::copies == 2 && HaloGeom<false>::copies == 3, "halo copies");

// LDS bytes of the resident weights (rounded up to whole 1 KiB copies) and of the kernel
__host__ __device__ constexpr int conv_halo_wbytes(int tr, int cin) {
  return ((tr * (9 * cin / 8 + 1) + 63) / 64) * 1024;
}
__host__ __device__ constexpr int conv_halo_lds_bytes(int tr, int cin, bool up2, int stages) {
  return conv_halo_wbytes(tr, cin) + stages * (up2 ? HaloGeom<true>::bytes : HaloGeom<false>::bytes) + tr * 4;
}

// read by the copies of halo pixels outside the image (chunk offsets stay inside it)
static __device__ __attribute__((aligned(1024))) unsigned char g_conv_zero_page[1024];

// the copies of a step landed, those of the stages_later (0 or 1) steps after it may be in flight;
// operations issued between them (stores) only make the wait stricter
template <int COPIES>
__device__ __forceinline__ void wait_copies(int stages_later) {
  static_assert(2 * COPIES < 16, "vmcnt encoding");
  if (stages_later == 0) __builtin_amdgcn_s_waitcnt(0x0F70);
  else __builtin_amdgcn_s_waitcnt(0x0F70 | COPIES);
}

constexpr int CH_WAVES = 8;  // one output row of the tile per wave

template <int TR, bool UP2, int STAGES>
__global__ void __launch_bounds__(512) conv_halo_kernel(const GemmP p) {
  using HG = HaloGeom<UP2>;
  constexpr int RW = conv_halo_rw(UP2), TH = HG::th;
  constexpr int NRB = TR / 16;  // MFMA row blocks (16 output channels each)
  constexpr int RUN = 4 * NRB;  // contiguous output channels per lane
  constexpr int COPIES = HG::copies;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lc = lane & 15, lg = lane >> 4;
  const int cin = p.cin;
  const int upr = 9 * cin / 8 + 1;  // 16-byte units per padded weight row
  const int wrowb = upr * 16;
  const int wunits = TR * upr;
  unsigned char* wl = lds;
  unsigned char* ring = lds + conv_halo_wbytes(TR, cin);
  float* btab = reinterpret_cast<float*>(ring + STAGES * HG::bytes);  // bias of the TR channels

  const int h = p.h, w = p.w;
  const int H = h << (UP2 ? 1 : 0), W = w << (UP2 ? 1 : 0);
  const int tiles_y = (H + TH - 1) / TH, tiles_x = (W + CH_TW - 1) / CH_TW;
  const int nimg = (int)(p.m / ((int64_t)H * W));
  const int ptiles = nimg * tiles_y * tiles_x;
  // XCD-aware (workgroup b runs on XCD b % 8; the grid is a multiple of 8 x ncol): the column
  // groups of a tile are adjacent workgroups of one XCD, so its halo comes into that XCD's L2 once
  // for all of them, and XCD x walks the contiguous tiles [T x / 8, T (x + 1) / 8), so the halo
  // rows that vertically adjacent tiles share are read there at about the same time. With the
  // column groups on different XCDs the 192 -> 64 conv (two groups) moved 1.8x its bytes.
  const int ncol = (int)cdiv(p.n, TR);
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int col = slot % ncol;
  const int kx = slot / ncol, per_xcd = gridDim.x / (8 * ncol);
  const int t_lo = (int)((int64_t)ptiles * xcd / 8), t_hi = (int)((int64_t)ptiles * (xcd + 1) / 8);
  const int ntiles = kx < t_hi - t_lo ? (t_hi - t_lo - kx + per_xcd - 1) / per_xcd : 0;
  const int nch = cin / CH_KC;
  const int nsteps = ntiles * nch;
  const unsigned char* X = (const unsigned char*)p.a;
  const unsigned char* Wt = (const unsigned char*)p.wt;
  if (ntiles == 0) return;  // before any copy is issued

  // ---- resident weights: unit v of the LDS region is row v / upr, 8 k at (v % upr) * 8; the
  // pad unit of a row and the units past the last row take any valid source
  for (int v0 = wave * 64; v0 < wunits; v0 += 64 * CH_WAVES) {
    const int v = v0 + lane;
    const int r = v / upr, j = v - r * upr;
    const bool real = r < TR && j < upr - 1;
    int64_t ch = (int64_t)col * TR + ((r & 15) >> 2) * RUN + (r >> 4) * 4 + (r & 3);
    if (!real) ch = (int64_t)col * TR;
    if (ch > p.n - 1) ch = p.n - 1;
    const unsigned char* src = Wt + (ch * 9 * cin + (real ? j : 0) * 8) * 2;
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)(wl + v0 * 16), 16, 0, 0);
  }

  // ---- bias table (0 for a missing bias or channels past n), copied with the weights
  if (wave == 0 && lane < TR) {
    const int64_t ch = (int64_t)col * TR + lane;
    if (p.bias && ch < p.n)
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(p.bias + ch),
                                       (__attribute__((address_space(3))) void*)btab, 4, 0, 0);
    else
      btab[lane] = 0.f;
  }

  // ---- halo copies: copy j of a wave moves the 16 halo pixels (wave + 8 j) * 16 .. + 15; lane
  // i fills pixel hp = (wave + 8 j) * 16 + i / 4, slot i % 4 with source unit slot ^ ((hp / 2) % 4)
  int hp_r[COPIES], hp_c[COPIES], hp_u[COPIES];
#pragma unroll
  for (int j = 0; j < COPIES; ++j) {
    const int hp = (wave + CH_WAVES * j) * 16 + (lane >> 2);
    hp_u[j] = (lane & 3) ^ ((hp >> 1) & 3);
    hp_r[j] = hp < HG::px ? hp / HG::cols : -1000000;  // padding slots: always outside the image
    hp_c[j] = hp < HG::px ? hp - (hp / HG::cols) * HG::cols : 0;
  }
  const unsigned char* hsrc[COPIES];
  int is_tile = 0, is_chunk = 0, is_stage = 0;
  auto set_issue_tile = [&]() __attribute__((always_inline)) {
    const int t = t_lo + kx + is_tile * per_xcd;
    const int img = t / (tiles_y * tiles_x);
    const int rem = t - img * tiles_y * tiles_x;
    const int ty = rem / tiles_x, tx = rem - (rem / tiles_x) * tiles_x;
    const int iy0 = UP2 ? ty * (TH / 2) - 1 : ty * TH - 1;  // input row of halo row 0
    const int ix0 = UP2 ? tx * (CH_TW / 2) - 1 : tx * CH_TW - 1;
#pragma unroll
    for (int j = 0; j < COPIES; ++j) {
      const int yy = iy0 + hp_r[j], xx = ix0 + hp_c[j];
      const bool ok = yy >= 0 && yy < h && xx >= 0 && xx < w;
      hsrc[j] = ok ? X + ((((int64_t)img * h + yy) * w + xx) * p.lda + hp_u[j] * 8) * 2
                   : g_conv_zero_page + hp_u[j] * 16;
    }
  };
  auto issue = [&]() __attribute__((always_inline)) {
    unsigned char* st = ring + is_stage * HG::bytes;
    const int cb = is_chunk * CH_KC * 2;  // byte offset of the chunk's channels (< 1024 - 64)
#pragma unroll
    for (int j = 0; j < COPIES; ++j)
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(hsrc[j] + cb),
                                       (__attribute__((address_space(3))) void*)(st + (wave + CH_WAVES * j) * 1024), 16,
                                       0, 0);
    is_stage = is_stage + 1 == STAGES ? 0 : is_stage + 1;
    if (++is_chunk == nch) {
      is_chunk = 0;
      ++is_tile;
      if (is_tile < ntiles) set_issue_tile();
    }
  };

  f32x4 acc[RW][2][NRB];  // [row of the wave][pixel block][16 channels]
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < NRB; ++b) acc[r][a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  set_issue_tile();
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < nsteps) issue();
  int s = 0, c_stage = 0;

  // ---- the outputs of the previous tile (bias, activation and scale applied), stored after the
  // next tile's first chunk has landed
  const int64_t run0 = (int64_t)col * TR + lg * RUN;
  const bool full_n = run0 + RUN <= p.n;
  float pend[RW][2][RUN];
  auto flush = [&](int tl) __attribute__((always_inline)) {
    const int t = t_lo + kx + tl * per_xcd;
    const int img = t / (tiles_y * tiles_x);
    const int rem = t - img * tiles_y * tiles_x;
    const int ty = rem / tiles_x, tx = rem - (rem / tiles_x) * tiles_x;
#pragma unroll
    for (int rp = 0; rp < 2 * RW; ++rp) {
      const int r = rp >> 1, pb = rp & 1;
      const int oy = ty * TH + RW * wave + r;
      const int ox = tx * CH_TW + pb * 16 + lc;
      if (oy >= H || ox >= W) continue;
      if (p.c_mode == CM_NCHW) {
        // channel planes [img][n][H][W] (output and residual): the 16 lanes of a channel store
        // 16 consecutive pixels of one row
        const int64_t hw = (int64_t)H * W;
        const int64_t o0 = ((int64_t)img * p.n + run0) * hw + (int64_t)oy * W + ox;
#pragma unroll
        for (int i = 0; i < RUN; ++i) {
          if (run0 + i >= p.n) continue;
          const int64_t o = o0 + i * hw;
          store1(p.c, p.c_dt, o, p.has_res ? pend[r][pb][i] + load1(p.res, p.r_dt, o) : pend[r][pb][i]);
        }
        continue;
      }
      const int64_t q = ((int64_t)img * H + oy) * W + ox;
      store_run<RUN>(p, pend[r][pb], q * p.ldc + run0, q * p.ldr + run0, run0, full_n);
    }
  };

  // one chunk step: wait for its copies and publish them, issue the copies STAGES - 1 steps
  // ahead, then all nine taps of the chunk. A tile's first step is peeled (it stores the previous
  // tile), so the held outputs are dead inside the chunk loop.
  auto step = [&](int kc, bool first, int tl) __attribute__((always_inline)) {
    const int later = (nsteps - 1 - s) < (STAGES - 2) ? (nsteps - 1 - s) : (STAGES - 2);
    wait_copies<COPIES>(later);  // the first: also the weights and the bias table, issued before
    barrier_keep_vm();
    if (first && tl > 0) flush(tl - 1);
    if (s + STAGES - 1 < nsteps) issue();
    const unsigned char* hb = ring + c_stage * HG::bytes;
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
      const int dy = tap / 3, dx = tap - (tap / 3) * 3;
      bf16x8 wf[NRB];
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb)
        wf[rb] = *reinterpret_cast<const bf16x8*>(wl + (rb * 16 + lc) * wrowb +
                                                  ((tap * cin + kc * CH_KC) / 8 + lg) * 16);
#pragma unroll
      for (int rp = 0; rp < 2 * RW; ++rp) {
        const int r = rp >> 1, pb = rp & 1;
        const int Y = RW * wave + r, Xo = pb * 16 + lc;
        const int hp = UP2 ? ((Y + dy + 1) >> 1) * HG::cols + ((Xo + dx + 1) >> 1) : (Y + dy) * HG::cols + Xo + dx;
        const bf16x8 af = *reinterpret_cast<const bf16x8*>(hb + hp * 64 + ((lg ^ ((hp >> 1) & 3)) * 16));
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) acc[r][pb][rb] = mfma_bf16(wf[rb], af, acc[r][pb][rb]);
      }
    }
    c_stage = c_stage + 1 == STAGES ? 0 : c_stage + 1;
    ++s;
  };

  for (int tl = 0; tl < ntiles; ++tl) {
    step(0, true, tl);
    for (int kc = 1; kc < nch; ++kc) step(kc, false, tl);

    // ---- epilogue of the tile up to the stores: bias (LDS table), activation, out_scale
#pragma unroll
    for (int rp = 0; rp < 2 * RW; ++rp) {
      const int r = rp >> 1, pb = rp & 1;
#pragma unroll
      for (int j = 0; j < NRB; ++j) {
        const f32x4 bb = *reinterpret_cast<const f32x4*>(btab + lg * RUN + j * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) pend[r][pb][j * 4 + i] = acc[r][pb][j][i] + bb[i];
        acc[r][pb][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      if (p.act == ACT_LRELU) {
#pragma unroll
        for (int i = 0; i < RUN; ++i) pend[r][pb][i] = pend[r][pb][i] >= 0.f ? pend[r][pb][i] : pend[r][pb][i] * p.slope;
      }
#pragma unroll
      for (int i = 0; i < RUN; ++i) pend[r][pb][i] *= p.out_scale;
    }
  }
  flush(ntiles - 1);
}

}  // namespace clarus
