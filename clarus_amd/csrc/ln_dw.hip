// Fused first half of a NAFNet block at width 64: clarus_hip_ln_gemm_dwconv (gfx950).
//
//   t   = LN(x) W1 + b1                          x [n, h, w, 64] bf16, W1 [64][128], t rounded to bf16
//   out = SG(dwconv3x3(t) + b_dw)                'same' zero padding, SimpleGate 128 -> 64
//
// Unfused, the 1x1 conv writes t (twice the width of x: 236 MB at 720 x 1280) and the depthwise
// conv reads it back; here t lives only in LDS. The arithmetic follows the two calls it replaces:
// the LayerNorm row (two-pass statistics, no affine) enters the products as bf16 hi + lo pairs
// (fp32-accurate), t is rounded to bf16 as the 1x1 conv stores it, and the depthwise conv sums
// bias, then taps (ky, kx) in fp32 (dwconv3x3_kernel's order), gates and rounds once.
//
// Tiles of LD_TR x LD_TW output pixels. A tile needs t on its (LD_TR + 2) x 32 halo pixels: one
// 32-pixel MFMA block per halo row, one halo row per wave (8 waves). Per tile:
//   * the halo's x rows (8 x 32 pixels x 128 B) travel global -> LDS by buffer copies into one of
//     two buffers, one tile ahead; pixels outside the image read as zeros through an
//     out-of-range offset;
//   * each wave computes t for its halo row on 32x32x16 MFMAs (W1 resident in LDS, packed so that
//     a lane's accumulators are two runs of 8 consecutive channels per 32-channel block), zeroes
//     the pixels outside the image (the depthwise conv's padding) and writes the row to the LDS
//     t tile;
//   * after a barrier, every thread computes 8 output channels of output pixels from the t tile
//     (9 taps x both gate halves, 16-byte LDS reads) and stores them.
// The 16-byte units of a t row (256 B per pixel) are XOR-swizzled by f(p) = 8 (p % 2) ^ (p / 2) % 8
// (those of an x row, 128 B, by p % 8):
// the 32 lanes writing one unit of 32 pixels hit 16 distinct bank groups (2-way), and the 16
// lanes of a depthwise read (2 adjacent pixels x 8 channel groups) hit 16.
// Every wave issues the same number of copies and stores per tile (stores of pixels outside the
// image go to an out-of-range offset), so the waits are exact vmcnt counts.
// No counterpart in the reference: it composes `linear` and `dwconv` (models/nafnet/__init__.py:
// 155-156), for hosts that run them back to back.
#include "capi.hpp"
#include "gemm_mfma32.hpp"

namespace clarus {

namespace {

constexpr int LD_C = 64, LD_M = 128;           // input / middle channels (output: LD_C)
constexpr int LD_TR = 6, LD_TW = 30;           // output tile
constexpr int LD_HR = LD_TR + 2, LD_HW = 32;   // halo tile: one MFMA block per row
constexpr int LD_WAVES = LD_HR;                // one halo row per wave
constexpr int LD_THREADS = 64 * LD_WAVES;
constexpr int LD_XB = LD_HR * LD_HW * LD_C * 2;          // x halo: 32 KiB
constexpr int LD_TB = LD_HR * LD_HW * LD_M * 2;          // t tile: 64 KiB
constexpr int LD_WB = LD_M * LD_C * 2;                   // packed W1: 16 KiB
constexpr int LD_TAB = (10 * LD_M + LD_M) * 4;           // taps [9][128], dw bias [128], b1 [128]
constexpr int LD_LDS = 2 * LD_XB + LD_TB + LD_WB + LD_TAB;
constexpr int LD_CPW = LD_XB / 1024 / LD_WAVES;          // x copies per wave per tile (4)
constexpr int LD_OUTS = LD_TR * LD_TW * (LD_C / 8);      // 8-channel outputs per tile (1440)
constexpr int LD_SPT = (LD_OUTS + LD_THREADS - 1) / LD_THREADS;  // stores per thread per tile (3)
static_assert(LD_LDS <= 160 * 1024 && LD_XB % (1024 * LD_WAVES) == 0, "LDS layout");

struct LdP {
  const bf16_t* x;    // [n, h, w, 64]
  const void* w1p;    // packed W1
  const float* b1;    // [128] or null
  const float* taps;  // [9][128]
  const float* dwb;   // [128] or null
  bf16_t* out;        // [n, h, w, 64]
  int n, h, w, tr, tc, ntiles;
  float ln_eps;
};

__device__ __forceinline__ int ld_swz(int p, int unit) { return unit ^ ((8 * (p & 1)) ^ ((p >> 1) & 7)); }

__global__ void __launch_bounds__(LD_THREADS) ln_dw_kernel(const LdP p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  unsigned char* xl = lds;                              // two x halo buffers
  unsigned char* tl = lds + 2 * LD_XB;                  // t tile
  unsigned char* wl = tl + LD_TB;                       // packed W1
  float* taps = reinterpret_cast<float*>(wl + LD_WB);  // [9][128]
  float* dwb = taps + 9 * LD_M;                         // [128]
  float* b1 = dwb + LD_M;                               // [128]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = p.h, W = p.w;
  const __amdgpu_buffer_rsrc_t xr = buf_rsrc_n(p.x, (uint32_t)((int64_t)p.n * H * W * LD_C * 2));
  const __amdgpu_buffer_rsrc_t orr = buf_rsrc_n(p.out, (uint32_t)((int64_t)p.n * H * W * LD_C * 2));
  constexpr uint32_t OOB = 0x80000000u;

  int t = blockIdx.x;
  if (t >= p.ntiles) return;
  // ---- W1 and the tables once
  for (int base = wave * 1024; base < LD_WB; base += LD_WAVES * 1024)
    __builtin_amdgcn_global_load_lds(
        (const __attribute__((address_space(1))) void*)((const unsigned char*)p.w1p + base + lane * 16),
        (__attribute__((address_space(3))) void*)(wl + base), 16, 0, 0);
  for (int i = tid; i < 11 * LD_M; i += LD_THREADS) {
    float v;
    if (i < 9 * LD_M) v = p.taps[i];
    else if (i < 10 * LD_M) v = p.dwb ? p.dwb[i - 9 * LD_M] : 0.f;
    else v = p.b1 ? p.b1[i - 10 * LD_M] : 0.f;
    taps[i] = v;
  }

  auto tile_of = [&](int tt, int& img, int& y0, int& x0) __attribute__((always_inline)) {
    x0 = (tt % p.tc) * LD_TW;
    const int r = tt / p.tc;
    y0 = (r % p.tr) * LD_TR;
    img = r / p.tr;
  };
  // x halo of tile tt into buffer b: wave w copies its 4 KiB share, lane l 16 bytes of pixel row
  // (1 KiB g + 16 l) / 128, unit ((1 KiB g + 16 l) / 16) % 8 (a halo pixel is 128 B of x)
  auto issue = [&](int tt, int b) __attribute__((always_inline)) {
    int img, y0, x0;
    tile_of(tt, img, y0, x0);
    int ln = lane;
    asm volatile("" : "+v"(ln));  // recomputed per tile: hoisted, the lane's copy offsets spilled
#pragma unroll
    for (int c = 0; c < LD_CPW; ++c) {
      const int g = wave * LD_CPW + c;                 // KiB of the halo buffer
      // LDS position (pixel hp, unit lane % 8) holds x unit (lane % 8) ^ (hp % 8): the 32 lanes reading
      // one unit of 32 pixels (128 B apart) spread over the bank groups
      const int hp = (g * 1024 + ln * 16) / (LD_C * 2), u = (ln & 7) ^ (hp & 7);
      const int yy = y0 - 1 + hp / LD_HW, xx = x0 - 1 + hp % LD_HW;
      const bool ok = yy >= 0 && yy < H && xx >= 0 && xx < W;
      const uint32_t off = ok ? (uint32_t)(((((int64_t)img * H + yy) * W + xx) * LD_C + u * 8) * 2) : OOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xr, (__attribute__((address_space(3))) void*)(xl + b * LD_XB + g * 1024), 16, off, 0, 0, 0);
    }
  };

  issue(t, 0);
  wait_vmem_all();  // W1 and the tables (and tile t's halo) have landed
  __syncthreads();
  for (int j = 0; t < p.ntiles; ++j, t += gridDim.x) {
    const int b = j & 1;
    if (j > 0) {
      // tile t's copies were issued during tile t - grid; only that tile's stores came after them
      wait_vmcnt<LD_SPT>();
      barrier_keep_vm();  // every wave's copies landed; the t tile of the last tile is free
    }
    const int tn = t + (int)gridDim.x;
    if (tn < p.ntiles) issue(tn, b ^ 1);  // the buffer last read in the previous tile's products
    int img, y0, x0;
    tile_of(t, img, y0, x0);

    // ---- t for halo row `wave`: LN(x) (hi + lo) . W1 + b1 on 32x32x16 MFMAs
    {
      int ln = lane;
      asm volatile("" : "+v"(ln));  // per tile, as below
      const int px = ln & 31, hf = ln >> 5;
      const unsigned char* xrow = xl + b * LD_XB + wave * (LD_HW * LD_C * 2) + px * (LD_C * 2);
      u32x4 q[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) q[s] = *reinterpret_cast<const u32x4*>(xrow + ((2 * s + hf) ^ (px & 7)) * 16);
      float xv[4][8];
      float sum = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          xv[s][2 * i] = __uint_as_float(q[s][i] << 16);
          xv[s][2 * i + 1] = __uint_as_float(q[s][i] & 0xffff0000u);
          sum += xv[s][2 * i] + xv[s][2 * i + 1];
        }
      sum += __shfl_xor(sum, 32, 64);
      const float mean = sum * (1.0f / LD_C);
      float ss = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          xv[s][i] -= mean;
          ss += xv[s][i] * xv[s][i];
        }
      ss += __shfl_xor(ss, 32, 64);
      const float rstd = rsqrtf(ss * (1.0f / LD_C) + p.ln_eps);
      bf16x8 xh[4], xlo[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        f32x8 a;
#pragma unroll
        for (int i = 0; i < 8; ++i) a.v[i] = xv[s][i] * rstd;
        split_bf16(a, xh[s], xlo[s]);
      }
      const int yy = y0 - 1 + wave, xx = x0 - 1 + px;
      const bool inside = yy >= 0 && yy < H && xx >= 0 && xx < W;
      unsigned char* trow = tl + (wave * LD_HW + px) * (LD_M * 2);
      const int hp = wave * LD_HW + px;  // halo pixel index (swizzle key)
#pragma unroll
      for (int T = 0; T < LD_M / 32; ++T) {
        // element j: middle channel 32 T + 16 (j / 8) + 8 hf + j % 8 (W1 rows permuted accordingly)
        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const f32x4 b0 = *reinterpret_cast<const f32x4*>(b1 + 32 * T + 16 * r + 8 * hf);
          const f32x4 b1v = *reinterpret_cast<const f32x4*>(b1 + 32 * T + 16 * r + 8 * hf + 4);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc[8 * r + i] = b0[i];
            acc[8 * r + 4 + i] = b1v[i];
          }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const bf16x8 wf = *reinterpret_cast<const bf16x8*>(wl + ((T * 4 + s) * 64 + ln) * 16);
          acc = mfma32_bf16(wf, xh[s], acc);
          acc = mfma32_bf16(wf, xlo[s], acc);
        }
        __builtin_amdgcn_sched_barrier(0);  // one 32-channel block's fragments at a time
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          u32x4 o;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            o[i] = inside ? ((unsigned)f32_to_bf16_bits(acc[8 * r + 2 * i]) |
                             ((unsigned)f32_to_bf16_bits(acc[8 * r + 2 * i + 1]) << 16))
                          : 0u;
          const int unit = (32 * T + 16 * r + 8 * hf) / 8;  // 16-byte unit of the 256-byte row
          *reinterpret_cast<u32x4*>(trow + ld_swz(hp, unit) * 16) = o;
        }
      }
    }
    barrier_keep_vm();  // the t tile is complete (LDS only: the next tile's copies stay in flight)

    // ---- depthwise 3x3 + SimpleGate. Thread tid < 8 RUNS: channel group cg = tid % 8 of the 3
    // output pixels (rows 3 rh .. 3 rh + 2, column ox) of run tid / 8 (rh = run / LD_TW, ox = run %
    // LD_TW). Per gate half its 5 x 3 input pixels are read once and each feeds up to 3 outputs,
    // and the taps of its channel group are read once (the per-output form read them for every
    // output and took most of the LDS bandwidth). Threads past 8 RUNS repeat the last run and store
    // out of range (every thread issues LD_SPT stores). Per output: bias, then taps (ky, kx).
    {
      constexpr int RUNS = LD_TW * (LD_TR / 3);
      static_assert(LD_TR % 3 == 0 && 8 * RUNS <= LD_THREADS && LD_SPT == 3, "depthwise runs");
      // the thread index laundered per tile: hoisted out of the tile loop, the LDS addresses
      // derived from it (15 inputs x 2 halves, 18 tap rows) stayed live and spilled
      int tq = tid;
      asm volatile("" : "+v"(tq));
      const int run0 = tq >> 3;
      const bool live = run0 < RUNS;
      const int run = live ? run0 : RUNS - 1;
      const int cg = tq & 7, rh = run / LD_TW, ox = run - rh * LD_TW;
      float g0[3][8];
      u32x4 o[3];
#pragma unroll
      for (int ou = 0; ou < 3; ++ou)
#pragma unroll
        for (int i = 0; i < 8; ++i) g0[ou][i] = 0.f;
#pragma unroll 1
      for (int h = 0; h < 2; ++h) {  // not unrolled: one half's 72 tap values live at a time
        float wv[9][8], acc[3][8];
#pragma unroll
        for (int tp = 0; tp < 9; ++tp) {
          const f32x4 w0 = *reinterpret_cast<const f32x4*>(taps + tp * LD_M + h * LD_C + cg * 8);
          const f32x4 w1 = *reinterpret_cast<const f32x4*>(taps + tp * LD_M + h * LD_C + cg * 8 + 4);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            wv[tp][i] = w0[i];
            wv[tp][4 + i] = w1[i];
          }
        }
        {
          const f32x4 v0 = *reinterpret_cast<const f32x4*>(dwb + h * LD_C + cg * 8);
          const f32x4 v1 = *reinterpret_cast<const f32x4*>(dwb + h * LD_C + cg * 8 + 4);
#pragma unroll
          for (int ou = 0; ou < 3; ++ou)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              acc[ou][i] = v0[i];
              acc[ou][4 + i] = v1[i];
            }
        }
#pragma unroll
        for (int r = 0; r < 5; ++r)
#pragma unroll
          for (int kx = 0; kx < 3; ++kx) {
            const int hp = (3 * rh + r) * LD_HW + ox + kx;
            const u32x4 v = *reinterpret_cast<const u32x4*>(tl + hp * (LD_M * 2) + ld_swz(hp, h * 8 + cg) * 16);
            float f[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              f[2 * i] = __uint_as_float(v[i] << 16);
              f[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
            }
#pragma unroll
            for (int ou = 0; ou < 3; ++ou) {
              const int ky = r - ou;
              if (ky < 0 || ky > 2) continue;
#pragma unroll
              for (int i = 0; i < 8; ++i) acc[ou][i] = fmaf(wv[ky * 3 + kx][i], f[i], acc[ou][i]);
            }
            if (kx == 2) __builtin_amdgcn_sched_barrier(0);  // one input row's reads at a time (spills)
          }
#pragma unroll
        for (int ou = 0; ou < 3; ++ou) {
#pragma unroll
          for (int i = 0; i < 4; ++i)  // after the second half: the gated outputs (g0 = the first)
            o[ou][i] = (unsigned)f32_to_bf16_bits(g0[ou][2 * i] * acc[ou][2 * i]) |
                       ((unsigned)f32_to_bf16_bits(g0[ou][2 * i + 1] * acc[ou][2 * i + 1]) << 16);
#pragma unroll
          for (int i = 0; i < 8; ++i) g0[ou][i] = acc[ou][i];
        }
      }
#pragma unroll
      for (int ou = 0; ou < 3; ++ou) {
        const int yy = y0 + 3 * rh + ou, xx = x0 + ox;
        const bool ok = live && yy < H && xx < W;
        const uint32_t off = ok ? (uint32_t)(((((int64_t)img * H + yy) * W + xx) * LD_C + cg * 8) * 2) : OOB;
        __builtin_amdgcn_raw_buffer_store_b128(o[ou], orr, off, 0, 0);
      }
    }
  }
  wait_vmem_all();
}

}  // namespace

}  // namespace clarus

using namespace clarus;

extern "C" int clarus_hip_ln_gemm_dwconv(const void* x, void* out, const void* w1p, const float* b1, const float* taps,
                                         const float* dwb, int64_t n, int64_t h, int64_t w, int64_t c, float ln_eps,
                                         void* stream) {
  clear_error();
  CLARUS_REQUIRE(x && out && w1p && taps, "ln_gemm_dwconv: null operand");
  CLARUS_REQUIRE(c == LD_C, "ln_gemm_dwconv: c = 64 only (c=%lld)", (long long)c);
  CLARUS_REQUIRE(n > 0 && h > 0 && w > 0, "ln_gemm_dwconv: empty problem");
  CLARUS_REQUIRE(n * h * w * LD_C * 2 < ((int64_t)1 << 31), "ln_gemm_dwconv: more than 2 GiB of activations");
  CLARUS_REQUIRE(aligned(x, 16) && aligned(out, 16) && aligned(w1p, 16) && aligned(taps, 16),
                 "ln_gemm_dwconv: 16-byte aligned operands");
  const char* xb = (const char*)x;
  const char* ob = (const char*)out;
  const int64_t bytes = n * h * w * LD_C * 2;
  CLARUS_REQUIRE(ob + bytes <= xb || xb + bytes <= ob, "ln_gemm_dwconv: out must not overlap x");
  LdP p{};
  p.x = (const bf16_t*)x; p.w1p = w1p; p.b1 = b1; p.taps = taps; p.dwb = dwb; p.out = (bf16_t*)out;
  p.n = (int)n; p.h = (int)h; p.w = (int)w;
  p.tr = (int)cdiv(h, LD_TR); p.tc = (int)cdiv(w, LD_TW);
  const int64_t ntiles = n * p.tr * p.tc;
  CLARUS_REQUIRE(ntiles < ((int64_t)1 << 31), "ln_gemm_dwconv: too many tiles");
  p.ntiles = (int)ntiles;
  p.ln_eps = ln_eps;
  static const bool attr = [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&ln_dw_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                              LD_LDS);
    return true;
  }();
  (void)attr;
  const int64_t nblk = ntiles < device_cus() ? ntiles : device_cus();
  note_kernel("ln_dw_kernel c=64");
  hipLaunchKernelGGL(ln_dw_kernel, dim3((unsigned)nblk), dim3(LD_THREADS), LD_LDS, (hipStream_t)stream, p);
  return check_launch("ln_gemm_dwconv");
}
