// 3x3 convolution (stride 1, zero padding 1, optional nearest-x2 input) on output tiles with an
// LDS halo, gfx950. bf16 input and weights, fp32 accumulation.
//
// The implicit-GEMM formulation reads every input pixel nine times (once per tap); here a
// workgroup instead
//   * keeps the weights of its TR output channels resident in LDS for the whole kernel
//     (W^T [TR][9 cin], rows padded by 16 bytes so the MFMA operand reads are conflict free),
//   * walks 8 x 32-pixel output tiles; per 32-input-channel chunk, the tile's input halo
//     ((8 + 2) x (32 + 2) pixels, or 6 x 18 at input resolution with the x2 upsample) arrives by
//     direct global->LDS copies into a ring of STAGES buffers; taps outside the image read a
//     zero page, so the padding costs no branches,
//   * and computes all nine taps from the halo: each of the 8 waves owns one output row (2
//     blocks of 16 pixels) and all TR channels, one bf16 MFMA (16 x 16 x 32) per (tap, pixel
//     block, 16 channels); two waves per SIMD hide each other's LDS latency.
// The K loop of a tile is one chunk per step with a single barrier; the epilogue (bias,
// LeakyReLU, out_scale, residual, 16-byte stores into a channel slice of the output) runs once
// per tile outside it, and the next tile's first halo is already in flight by then. NCHW fp32
// output (c_mode NCHW, the NAFNet ending conv with its global residual) is stored per channel
// plane; TR = 16 serves narrow outputs (cout <= 16, e.g. 3 image channels).
#pragma once

#include "gemm_lds.hpp"

namespace clarus {

constexpr int CH_TH = 8;   // output tile rows
constexpr int CH_TW = 32;  // output tile columns
constexpr int CH_KC = 32;  // input channels per chunk

template <bool UP2>
struct HaloGeom {
  static constexpr int rows = UP2 ? CH_TH / 2 + 2 : CH_TH + 2;  // 6 / 10
  static constexpr int cols = UP2 ? CH_TW / 2 + 2 : CH_TW + 2;  // 18 / 34
  static constexpr int px = rows * cols;                          // 108 / 340
  static constexpr int px_pad = UP2 ? 128 : 384;                  // a whole number of 16-pixel copies per wave
  static constexpr int bytes = px_pad * 64;                       // 32 bf16 channels per pixel
  static constexpr int copies = px_pad / 128;                     // 16-byte copies per lane per stage (8 waves)
};

// LDS bytes of the resident weights (rounded up to whole 1 KiB copies) and of the kernel
__host__ __device__ constexpr int conv_halo_wbytes(int tr, int cin) {
  return ((tr * (9 * cin / 8 + 1) + 63) / 64) * 1024;
}
__host__ __device__ constexpr int conv_halo_lds_bytes(int tr, int cin, bool up2, int stages) {
  return conv_halo_wbytes(tr, cin) + stages * (up2 ? HaloGeom<true>::bytes : HaloGeom<false>::bytes);
}

// read by the copies of halo pixels outside the image (chunk offsets stay inside it)
static __device__ __attribute__((aligned(1024))) unsigned char g_conv_zero_page[1024];

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

  const int h = p.h, w = p.w;
  const int H = h << (UP2 ? 1 : 0), W = w << (UP2 ? 1 : 0);
  const int tiles_y = (H + CH_TH - 1) / CH_TH, tiles_x = (W + CH_TW - 1) / CH_TW;
  const int nimg = (int)(p.m / ((int64_t)H * W));
  const int ptiles = nimg * tiles_y * tiles_x;
  const int ncol = (int)cdiv(p.n, TR);
  const int col = blockIdx.x % ncol;
  const int wg = blockIdx.x / ncol, nwg = gridDim.x / ncol;
  const int ntiles = wg < ptiles ? (ptiles - wg + nwg - 1) / nwg : 0;
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
    const int t = wg + is_tile * nwg;
    const int img = t / (tiles_y * tiles_x);
    const int rem = t - img * tiles_y * tiles_x;
    const int ty = rem / tiles_x, tx = rem - (rem / tiles_x) * tiles_x;
    const int iy0 = UP2 ? ty * (CH_TH / 2) - 1 : ty * CH_TH - 1;  // input row of halo row 0
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

  f32x4 acc[2][NRB];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < NRB; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  set_issue_tile();
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < nsteps) issue();
  int s = 0, c_stage = 0;

  for (int tl = 0; tl < ntiles; ++tl) {
    for (int kc = 0; kc < nch; ++kc, ++s) {
      const int later = (nsteps - 1 - s) < (STAGES - 2) ? (nsteps - 1 - s) : (STAGES - 2);
      wait_copies<COPIES>(kc == 0 ? 0 : later);  // a tile's first chunk: everything (weights, epilogue)
      barrier_keep_vm();
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
        for (int pb = 0; pb < 2; ++pb) {
          const int Y = wave, Xo = pb * 16 + lc;
          const int hp = UP2 ? ((Y + dy + 1) >> 1) * HG::cols + ((Xo + dx + 1) >> 1) : (Y + dy) * HG::cols + Xo + dx;
          const bf16x8 af = *reinterpret_cast<const bf16x8*>(hb + hp * 64 + ((lg ^ ((hp >> 1) & 3)) * 16));
#pragma unroll
          for (int rb = 0; rb < NRB; ++rb) acc[pb][rb] = mfma_bf16(wf[rb], af, acc[pb][rb]);
        }
      }
      c_stage = c_stage + 1 == STAGES ? 0 : c_stage + 1;
    }

    // ---- epilogue of the tile
    {
      const int t = wg + tl * nwg;
      const int img = t / (tiles_y * tiles_x);
      const int rem = t - img * tiles_y * tiles_x;
      const int ty = rem / tiles_x, tx = rem - (rem / tiles_x) * tiles_x;
      const int64_t run0 = (int64_t)col * TR + lg * RUN;
      const bool full_n = run0 + RUN <= p.n;
      float b1[RUN];
#pragma unroll
      for (int i = 0; i < RUN; ++i) b1[i] = (p.bias && run0 + i < p.n) ? p.bias[run0 + i] : 0.f;
#pragma unroll
      for (int pb = 0; pb < 2; ++pb) {
        const int oy = ty * CH_TH + wave;
        const int ox = tx * CH_TW + pb * 16 + lc;
        float v[RUN];
#pragma unroll
        for (int j = 0; j < NRB; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) v[j * 4 + i] = acc[pb][j][i] + b1[j * 4 + i];
#pragma unroll
        for (int j = 0; j < NRB; ++j) acc[pb][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (oy >= H || ox >= W) continue;
        if (p.act == ACT_LRELU) {
#pragma unroll
          for (int i = 0; i < RUN; ++i) v[i] = v[i] >= 0.f ? v[i] : v[i] * p.slope;
        }
#pragma unroll
        for (int i = 0; i < RUN; ++i) v[i] *= p.out_scale;
        if (p.c_mode == CM_NCHW) {
          // channel planes [img][n][H][W] (output and residual): the 16 lanes of a channel store
          // 16 consecutive pixels of one row
          const int64_t hw = (int64_t)H * W;
          const int64_t o0 = ((int64_t)img * p.n + run0) * hw + (int64_t)oy * W + ox;
#pragma unroll
          for (int i = 0; i < RUN; ++i) {
            if (run0 + i >= p.n) continue;
            const int64_t o = o0 + i * hw;
            store1(p.c, p.c_dt, o, p.has_res ? v[i] + load1(p.res, p.r_dt, o) : v[i]);
          }
          continue;
        }
        const int64_t q = ((int64_t)img * H + oy) * W + ox;
        store_run<RUN>(p, v, q * p.ldc + run0, q * p.ldr + run0, run0, full_n);
      }
    }
  }
}

}  // namespace clarus
