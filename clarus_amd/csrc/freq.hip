// Per-8x8-patch DFT operators of FFTformer as dense real products on fp32 MFMA (gfx950).
//
// A patch of one channel is a 64-vector x (pixel r * 8 + s). With the 80 x 64 real matrix
// Fwd (rows 2b / 2b + 1 = Re / Im of rfft2 bin b = u * 5 + v) and the 64 x 80 matrix Inv
// (column j = irfft2, s=(8, 8), of the unit coefficient j, which encodes irfft2's handling of
// non-Hermitian v = 0 / v = 4 columns):
//   patch_filter : y = Inv . (g_c * (Fwd . x))           (+ residual)
//   patch_corr   : y = Inv . (Fwd q (*) Fwd k)           (complex product per bin)
// Work unit = (patch, 16 channels), one wave. The forward product D1 = Fwd . X has the 80
// coefficients as MFMA rows and the 16 channels as columns; its accumulator registers are
// reused directly as the B operand of the inverse product (the k index of instruction
// (rb, j) is coefficient 16 rb + 4 (l / 16) + j, and Inv is read with the same mapping), so
// nothing goes through LDS except the two constant matrices.
#include "capi.hpp"
#include "common.hpp"

namespace clarus {

constexpr int NCOEF = 80;

struct FreqP {
  const void* x;
  const float* fwd;
  const float* inv;
  const float* gain;  // patch_filter: [c][80]
  const void* res;
  void* out;
  int64_t sn, sh, sw;  // x strides (elements): batch, row, pixel
  int64_t batch, h, w, c;
  int64_t units;       // patches * channel blocks
  int x_dt, r_dt, o_dt;
  int corr;            // 0 filter, 1 correlation
};

// stage Fwd [80][64] and Inv [64][80] into LDS (padded rows: no bank conflicts)
constexpr int FROW = 64 + 4;
constexpr int IROW = 80 + 4;

template <int XDT>
__global__ void __launch_bounds__(256) patch_kernel(const FreqP p) {
  __shared__ __attribute__((aligned(16))) float fw[NCOEF * FROW];
  __shared__ __attribute__((aligned(16))) float iv[64 * IROW];
  for (int e = threadIdx.x; e < NCOEF * 64; e += 256) fw[(e / 64) * FROW + (e % 64)] = p.fwd[e];
  for (int e = threadIdx.x; e < 64 * NCOEF; e += 256) iv[(e / NCOEF) * IROW + (e % NCOEF)] = p.inv[e];
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lc = lane & 15, lg = lane >> 4;
  const int64_t ph = cdiv(p.h, 8), pw = cdiv(p.w, 8);
  const int64_t cblocks = cdiv(p.c, 16);
  constexpr int XES = (XDT == DT_BF16) ? 2 : 4;

  for (int64_t u = (int64_t)blockIdx.x * 4 + wave; u < p.units; u += (int64_t)gridDim.x * 4) {
    const int64_t cb = u % cblocks;
    const int64_t patch = u / cblocks;
    const int64_t n = patch / (ph * pw);
    const int64_t rem = patch - n * ph * pw;
    const int64_t py = rem / pw, px = rem - (rem / pw) * pw;
    const int64_t ch = cb * 16 + lc;
    const bool cval = ch < p.c;

    // x value of pixel i (0..63) of this patch for this lane's channel; reflect padding at the
    // bottom / right edge (torch F.pad mode="reflect": index 2 (L - 1) - i past the end)
    auto xoff = [&](int i, int64_t coff) -> int64_t {
      int64_t yy = py * 8 + (i >> 3), xx = px * 8 + (i & 7);
      if (yy >= p.h) yy = 2 * (p.h - 1) - yy;
      if (xx >= p.w) xx = 2 * (p.w - 1) - xx;
      return n * p.sn + yy * p.sh + xx * p.sw + coff;
    };

    // ---- forward: D1[rb] (rows = coefficients 16 rb + 4 lg + j, column = channel lc)
    f32x4 d1[5], d2[5];
#pragma unroll
    for (int rb = 0; rb < 5; ++rb) d1[rb] = d2[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {  // 32 pixels per step, lane: pixels kb*32 + 8 lg + s
      float xv[8], kv[8];
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int i = kb * 32 + lg * 8 + s;
        xv[s] = cval ? load1(p.x, XDT, xoff(i, ch)) : 0.f;
        if (p.corr) kv[s] = cval ? load1(p.x, XDT, xoff(i, p.c + ch)) : 0.f;
      }
#pragma unroll
      for (int rb = 0; rb < 5; ++rb) {
        const float* fr = fw + (rb * 16 + lc) * FROW + kb * 32 + lg * 8;
        const f32x4 f0 = *reinterpret_cast<const f32x4*>(fr);
        const f32x4 f1 = *reinterpret_cast<const f32x4*>(fr + 4);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          d1[rb] = mfma_f32(f0[s], xv[s], d1[rb]);
          if (p.corr) d2[rb] = mfma_f32(f0[s], kv[s], d2[rb]);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          d1[rb] = mfma_f32(f1[s], xv[4 + s], d1[rb]);
          if (p.corr) d2[rb] = mfma_f32(f1[s], kv[4 + s], d2[rb]);
        }
      }
    }
    // ---- per-coefficient operation (lane holds coefficients 16 rb + 4 lg + j, j = 0..3;
    // (j, j+1) for j = 0, 2 are the Re / Im pair of one bin)
#pragma unroll
    for (int rb = 0; rb < 5; ++rb) {
      if (p.corr) {
        const float ar = d1[rb][0], ai = d1[rb][1], br = d2[rb][0], bi = d2[rb][1];
        const float cr = d1[rb][2], ci = d1[rb][3], dr = d2[rb][2], di = d2[rb][3];
        d1[rb][0] = ar * br - ai * bi;
        d1[rb][1] = ar * bi + ai * br;
        d1[rb][2] = cr * dr - ci * di;
        d1[rb][3] = cr * di + ci * dr;
      } else if (cval) {
        const f32x4 g = *reinterpret_cast<const f32x4*>(p.gain + ch * NCOEF + rb * 16 + lg * 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) d1[rb][j] *= g[j];
      }
    }
    // ---- inverse: y[ob] rows = pixels 16 ob + 4 lg + j, column = channel
#pragma unroll
    for (int ob = 0; ob < 4; ++ob) {
      f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int rb = 0; rb < 5; ++rb) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(iv + (ob * 16 + lc) * IROW + rb * 16 + lg * 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) y = mfma_f32(a[j], d1[rb][j], y);
      }
      if (!cval) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = ob * 16 + lg * 4 + j;
        const int64_t yy = py * 8 + (i >> 3), xx = px * 8 + (i & 7);
        if (yy >= p.h || xx >= p.w) continue;
        const int64_t o = ((n * p.h + yy) * p.w + xx) * p.c + ch;  // out / residual contiguous
        float v = y[j];
        if (p.res) v += load1(p.res, p.r_dt, o);
        store1(p.out, p.o_dt, o, v);
      }
    }
  }
}

static int launch_patch(FreqP& p, hipStream_t s, const char* what) {
  const int64_t patches = p.batch * cdiv(p.h, 8) * cdiv(p.w, 8);
  p.units = patches * cdiv(p.c, 16);
  int64_t blocks = cdiv(p.units, 4);
  if (blocks > 4096) blocks = 4096;
  if (p.x_dt == DT_BF16)
    hipLaunchKernelGGL(patch_kernel<DT_BF16>, dim3((unsigned)blocks), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(patch_kernel<DT_F32>, dim3((unsigned)blocks), dim3(256), 0, s, p);
  return check_launch(what);
}

}  // namespace clarus

using namespace clarus;

extern "C" int clarus_hip_patch_filter(const void* x, int32_t x_dtype, int64_t ldx, const float* fwd,
                                       const float* inv, const float* gain, const void* res, int32_t r_dtype,
                                       void* out, int32_t o_dtype, int64_t batch, int64_t h, int64_t w, int64_t c,
                                       void* stream) {
  clear_error();
  CLARUS_REQUIRE(x && fwd && inv && gain && out, "patch_filter: null operand");
  CLARUS_REQUIRE(batch > 0 && h > 0 && w > 0 && c > 0 && ldx >= c, "patch_filter: bad sizes");
  CLARUS_REQUIRE((x_dtype == DT_F32 || x_dtype == DT_BF16) && (o_dtype == DT_F32 || o_dtype == DT_BF16),
                 "patch_filter: bad dtype");
  CLARUS_REQUIRE((h % 8 == 0 || h > (8 - h % 8)) && (w % 8 == 0 || w > (8 - w % 8)),
                 "patch_filter: reflect padding to a multiple of 8 needs h, w larger than the pad");
  CLARUS_REQUIRE(aligned(gain, 16) && aligned(fwd, 16) && aligned(inv, 16), "patch_filter: matrix alignment");
  if (res) CLARUS_REQUIRE(r_dtype == DT_F32 || r_dtype == DT_BF16, "patch_filter: bad residual dtype");
  FreqP p{};
  p.x = x; p.fwd = fwd; p.inv = inv; p.gain = gain; p.res = res; p.out = out;
  p.sn = h * w * ldx; p.sh = w * ldx; p.sw = ldx;
  p.batch = batch; p.h = h; p.w = w; p.c = c;
  p.x_dt = x_dtype; p.r_dt = r_dtype; p.o_dt = o_dtype; p.corr = 0;
  return launch_patch(p, (hipStream_t)stream, "patch_filter");
}

extern "C" int clarus_hip_patch_corr(const void* x, int32_t x_dtype, int64_t sn, int64_t sh, int64_t sw,
                                     const float* fwd, const float* inv, float* out, int64_t batch, int64_t h,
                                     int64_t w, int64_t c, void* stream) {
  clear_error();
  CLARUS_REQUIRE(x && fwd && inv && out, "patch_corr: null operand");
  CLARUS_REQUIRE(batch > 0 && h > 0 && w > 0 && c > 0 && h % 8 == 0 && w % 8 == 0,
                 "patch_corr: h, w must be multiples of 8");
  CLARUS_REQUIRE(x_dtype == DT_F32 || x_dtype == DT_BF16, "patch_corr: bad dtype");
  CLARUS_REQUIRE(aligned(fwd, 16) && aligned(inv, 16), "patch_corr: matrix alignment");
  FreqP p{};
  p.x = x; p.fwd = fwd; p.inv = inv; p.gain = nullptr; p.res = nullptr; p.out = out;
  p.sn = sn; p.sh = sh; p.sw = sw;
  p.batch = batch; p.h = h; p.w = w; p.c = c;
  p.x_dt = x_dtype; p.r_dt = DT_F32; p.o_dt = DT_F32; p.corr = 1;
  return launch_patch(p, (hipStream_t)stream, "patch_corr");
}
