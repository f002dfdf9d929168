// Per-8x8-patch DFT operators of FFTformer as dense real products on MFMA (gfx950).
//
// A patch of one channel is a 64-vector x (pixel r * 8 + s). With the 80 x 64 real matrix
// Fwd (rows 2b / 2b + 1 = Re / Im of rfft2 bin b = u * 5 + v) and the 64 x 80 matrix Inv
// (column j = irfft2, s=(8, 8), of the unit coefficient j, which encodes irfft2's handling of
// non-Hermitian v = 0 / v = 4 columns):
//   patch_filter : y = Inv . (g_c * (Fwd . x))           (+ residual)
//   patch_corr   : y = Inv . (Fwd q (*) Fwd k)           (complex product per bin)
// Work unit = (patch, 16 channels), one wave. The forward product D1 = Fwd . X has the 80
// coefficients as MFMA rows and the 16 channels as columns; its accumulator registers are
// reused directly as the B operand of the inverse product (Inv is staged with its columns in
// the order a lane holds the coefficients), so nothing goes through LDS except the two
// constant matrices. fp32 values enter bf16 MFMAs as hi + lo pairs (x = hi + lo to 2^-18
// relative) with three products per block (hi hi + hi lo + lo hi; the dropped lo lo term is
// 2^-18 relative), fp32 accumulation.
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
  int small_offsets;   // in-patch offsets (7 rows, 7 pixels, 2 c channels) fit 31 bits
};

// LDS copies of the operators as bf16 hi / lo pairs (x = hi + lo to 2^-18 relative):
//   Fwd [80 rows][64 k]                     (A operand of the forward product)
//   Inv [64 rows][96 k], k permuted: column 32 kb + 8 g + i holds coefficient
//       16 (2 kb + i / 4) + 4 g + i % 4 (zero past 80), the order in which a lane holds the
//       forward accumulators, so they are the B operand of the inverse product as they stand.
constexpr int FROWB = (64 + 8) * 2;   // bytes per Fwd row (+16 B pad)
constexpr int IROWB = (96 + 8) * 2;   // bytes per Inv row
constexpr int FBYTES = NCOEF * FROWB;
constexpr int IBYTES = 64 * IROWB;

__device__ __forceinline__ bf16x8 lds8(const unsigned char* p) { return *reinterpret_cast<const bf16x8*>(p); }

template <int XDT, bool CORR>
__global__ void __launch_bounds__(256) patch_kernel(const FreqP p) {
  __shared__ __attribute__((aligned(16))) unsigned char fw[2 * FBYTES];  // hi, then lo
  __shared__ __attribute__((aligned(16))) unsigned char iv[2 * IBYTES];
  // staging with 16-byte loads: 4 consecutive k of one row per step, split into 8-byte hi / lo
  auto put4 = [](unsigned char* dhi, unsigned char* dlo, const f32x4 f) __attribute__((always_inline)) {
    bf16_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      h[i] = (bf16_t)f[i];
      l[i] = (bf16_t)(f[i] - (float)h[i]);
    }
    *reinterpret_cast<u32x2*>(dhi) = u32x2{(unsigned)__builtin_bit_cast(unsigned short, h[0]) |
                                               ((unsigned)__builtin_bit_cast(unsigned short, h[1]) << 16),
                                           (unsigned)__builtin_bit_cast(unsigned short, h[2]) |
                                               ((unsigned)__builtin_bit_cast(unsigned short, h[3]) << 16)};
    *reinterpret_cast<u32x2*>(dlo) = u32x2{(unsigned)__builtin_bit_cast(unsigned short, l[0]) |
                                               ((unsigned)__builtin_bit_cast(unsigned short, l[1]) << 16),
                                           (unsigned)__builtin_bit_cast(unsigned short, l[2]) |
                                               ((unsigned)__builtin_bit_cast(unsigned short, l[3]) << 16)};
  };
  for (int e = threadIdx.x; e < NCOEF * 16; e += 256) {  // Fwd [80][64]: 16 groups of 4 per row
    const int r = e >> 4, k = (e & 15) * 4;
    const f32x4 f = *reinterpret_cast<const f32x4*>(p.fwd + r * 64 + k);
    put4(fw + r * FROWB + k * 2, fw + FBYTES + r * FROWB + k * 2, f);
  }
  for (int e = threadIdx.x; e < 64 * 24; e += 256) {  // Inv [64][96 permuted]: 24 groups of 4 per row
    const int r = e / 24, kk = (e - (e / 24) * 24) * 4;
    const int kb = kk >> 5, g = (kk >> 3) & 3, i = kk & 7;  // i = 0 or 4
    const int coef = 16 * (2 * kb + (i >> 2)) + 4 * g;       // 4 consecutive coefficients
    const f32x4 f = coef < NCOEF ? *reinterpret_cast<const f32x4*>(p.inv + r * NCOEF + coef)
                                 : f32x4{0.f, 0.f, 0.f, 0.f};
    put4(iv + r * IROWB + kk * 2, iv + IBYTES + r * IROWB + kk * 2, f);
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lc = lane & 15, lg = lane >> 4;
  const int ph = (int)cdiv(p.h, 8), pw = (int)cdiv(p.w, 8);
  const int cblocks = (int)cdiv(p.c, 16);
  const int H = (int)p.h, W = (int)p.w;
  constexpr int XES = (XDT == DT_BF16) ? 2 : 4;

  for (int64_t u = (int64_t)blockIdx.x * 4 + wave; u < p.units; u += (int64_t)gridDim.x * 4) {
    // compiler-only barrier: re-read the operator fragments from LDS per unit instead of
    // hoisting all of them into registers (which would cost occupancy)
    asm volatile("" ::: "memory");
    const int cb = (int)(u % cblocks);
    const int64_t patch = u / cblocks;
    const int64_t n = patch / ((int64_t)ph * pw);
    const int rem = (int)(patch - n * ph * pw);
    const int py = rem / pw, px = rem - (rem / pw) * pw;
    const int64_t ch = (int64_t)cb * 16 + lc;
    const bool cval = ch < p.c;
    const int64_t chl = cval ? ch : 0;

    // this lane's 8 pixels of k-block kb: row 4 kb + lg (0..7), columns 0..7 of the patch;
    // reflect padding at the bottom / right edge (torch F.pad mode="reflect"). Interior patches
    // (uniform per wave) address with 32-bit offsets from the patch origin.
    const bool interior = py * 8 + 8 <= H && px * 8 + 8 <= W;
    bf16x8 xh[2], xl[2], kh[2], kl[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      f32x8 xv, kv;
      if (interior && p.small_offsets) {
        const unsigned char* o0 = (const unsigned char*)p.x +
                                  (n * p.sn + (int64_t)(py * 8) * p.sh + (int64_t)(px * 8) * p.sw + chl) * XES;
        const int rowo = (kb * 4 + lg) * (int)p.sh;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const int o = rowo + s * (int)p.sw;
          xv.v[s] = cval ? (XDT == DT_BF16 ? bf16_to_f32(*reinterpret_cast<const unsigned short*>(o0 + (int64_t)o * 2))
                                           : *reinterpret_cast<const float*>(o0 + (int64_t)o * 4))
                         : 0.f;
          if constexpr (CORR)
            kv.v[s] = cval ? (XDT == DT_BF16
                                  ? bf16_to_f32(*reinterpret_cast<const unsigned short*>(o0 + ((int64_t)o + p.c) * 2))
                                  : *reinterpret_cast<const float*>(o0 + ((int64_t)o + p.c) * 4))
                           : 0.f;
        }
      } else {
        int yy = py * 8 + kb * 4 + lg;
        if (yy >= H) yy = 2 * (H - 1) - yy;
        const int64_t rowoff = n * p.sn + (int64_t)yy * p.sh;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          int xx = px * 8 + s;
          if (xx >= W) xx = 2 * (W - 1) - xx;
          const int64_t o = rowoff + (int64_t)xx * p.sw;
          xv.v[s] = cval ? load1(p.x, XDT, o + chl) : 0.f;
          if constexpr (CORR) kv.v[s] = cval ? load1(p.x, XDT, o + p.c + chl) : 0.f;
        }
      }
      split_bf16(xv, xh[kb], xl[kb]);
      if constexpr (CORR) split_bf16(kv, kh[kb], kl[kb]);
    }

    // ---- forward: d1[rb] rows = coefficients 16 rb + 4 lg + j, column = channel lc
    f32x4 d1[5], d2[CORR ? 5 : 1];
#pragma unroll
    for (int rb = 0; rb < 5; ++rb) {
      d1[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (CORR) d2[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int off = (rb * 16 + lc) * FROWB + (kb * 32 + lg * 8) * 2;
        const bf16x8 fh = lds8(fw + off), fl = lds8(fw + FBYTES + off);
        d1[rb] = mfma_bf16(fh, xh[kb], d1[rb]);
        d1[rb] = mfma_bf16(fh, xl[kb], d1[rb]);
        d1[rb] = mfma_bf16(fl, xh[kb], d1[rb]);
        if constexpr (CORR) {
          d2[rb] = mfma_bf16(fh, kh[kb], d2[rb]);
          d2[rb] = mfma_bf16(fh, kl[kb], d2[rb]);
          d2[rb] = mfma_bf16(fl, kh[kb], d2[rb]);
        }
      }
    }
    // ---- per-coefficient operation ((j, j + 1), j = 0, 2 are the Re / Im pair of one bin)
#pragma unroll
    for (int rb = 0; rb < 5; ++rb) {
      if constexpr (CORR) {
        const float ar = d1[rb][0], ai = d1[rb][1], br = d2[rb][0], bi = d2[rb][1];
        const float cr = d1[rb][2], ci = d1[rb][3], dr = d2[rb][2], di = d2[rb][3];
        d1[rb][0] = ar * br - ai * bi;
        d1[rb][1] = ar * bi + ai * br;
        d1[rb][2] = cr * dr - ci * di;
        d1[rb][3] = cr * di + ci * dr;
      } else {
        const f32x4 g = cval ? *reinterpret_cast<const f32x4*>(p.gain + chl * NCOEF + rb * 16 + lg * 4)
                             : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) d1[rb][j] *= g[j];
      }
    }
    // the B operand of the inverse: k-block kb2 = coefficient row blocks 2 kb2, 2 kb2 + 1
    bf16x8 dh[3], dl[3];
#pragma unroll
    for (int kb2 = 0; kb2 < 3; ++kb2) {
      f32x8 dv;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        dv.v[j] = d1[2 * kb2][j];
        dv.v[4 + j] = (2 * kb2 + 1 < 5) ? d1[2 * kb2 + 1 < 5 ? 2 * kb2 + 1 : 0][j] : 0.f;
      }
      split_bf16(dv, dh[kb2], dl[kb2]);
    }
    // ---- inverse: y[ob] rows = pixels 16 ob + 4 lg + j (patch row 2 ob + lg / 2), column = channel
#pragma unroll
    for (int ob = 0; ob < 4; ++ob) {
      f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb2 = 0; kb2 < 3; ++kb2) {
        const int off = (ob * 16 + lc) * IROWB + (kb2 * 32 + lg * 8) * 2;
        const bf16x8 ih = lds8(iv + off), il = lds8(iv + IBYTES + off);
        y = mfma_bf16(ih, dh[kb2], y);
        y = mfma_bf16(ih, dl[kb2], y);
        y = mfma_bf16(il, dh[kb2], y);
      }
      if (!cval) continue;
      const int pi0 = ob * 16 + lg * 4;  // pixels pi0 .. pi0 + 3: one patch row, 4 columns
      const int yy = py * 8 + (pi0 >> 3);
      if (yy >= H) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int xx = px * 8 + (pi0 & 7) + j;
        if (xx >= W) continue;
        const int64_t o = ((n * H + yy) * W + xx) * p.c + ch;  // out / residual contiguous
        float v = y[j];
        if (p.res) v += load1(p.res, p.r_dt, o);
        store1(p.out, p.o_dt, o, v);
      }
    }
  }
}

static int launch_patch(FreqP& p, hipStream_t s, const char* what) {
  p.small_offsets = (7 * p.sh + 7 * p.sw + 2 * p.c) < ((int64_t)1 << 31) && p.sh < ((int64_t)1 << 31) &&
                    p.sw < ((int64_t)1 << 31);
  const int64_t patches = p.batch * cdiv(p.h, 8) * cdiv(p.w, 8);
  p.units = patches * cdiv(p.c, 16);
  // persistent: ~3 resident workgroups per CU (the LDS operator copies), so each stages the
  // matrices once for many units
  int64_t blocks = cdiv(p.units, 4);
  if (blocks > 768) blocks = 768;
  const dim3 g((unsigned)blocks);
  if (p.corr) {
    if (p.x_dt == DT_BF16) hipLaunchKernelGGL((patch_kernel<DT_BF16, true>), g, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((patch_kernel<DT_F32, true>), g, dim3(256), 0, s, p);
  } else {
    if (p.x_dt == DT_BF16) hipLaunchKernelGGL((patch_kernel<DT_BF16, false>), g, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((patch_kernel<DT_F32, false>), g, dim3(256), 0, s, p);
  }
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
