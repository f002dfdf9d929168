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
#include <type_traits>

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

// 4 consecutive fp32 values written to LDS as 8-byte bf16 hi / lo runs (x = hi + lo)
__device__ __forceinline__ void put4_split(unsigned char* dhi, unsigned char* dlo, const f32x4 f) {
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
}

// Inv staged as the B-order operand of the inverse product (shared by both kernels)
__device__ __forceinline__ void stage_inv(unsigned char* iv, const float* inv) {
  for (int e = threadIdx.x; e < 64 * 24; e += blockDim.x) {  // Inv [64][96 permuted]: 24 groups of 4 per row
    const int r = e / 24, kk = (e - (e / 24) * 24) * 4;
    const int kb = kk >> 5, g = (kk >> 3) & 3, i = kk & 7;  // i = 0 or 4
    const int coef = 16 * (2 * kb + (i >> 2)) + 4 * g;       // 4 consecutive coefficients
    const f32x4 f = coef < NCOEF ? *reinterpret_cast<const f32x4*>(inv + r * NCOEF + coef)
                                 : f32x4{0.f, 0.f, 0.f, 0.f};
    put4_split(iv + r * IROWB + kk * 2, iv + IBYTES + r * IROWB + kk * 2, f);
  }
}

// A work unit's position: channel block cb, patch column px, row py, image n (wave-uniform)
struct PatchPos {
  int cb, px, py;
  int64_t n;
};

// 8 waves per workgroup share one LDS copy of the operators (50 KiB): two workgroups per CU,
// 4 waves per SIMD (at most 128 VGPRs), so more units' loads are in flight per SIMD
constexpr int PK_WAVES = 8;
template <int XDT, bool CORR>
__global__ void __launch_bounds__(64 * PK_WAVES) __attribute__((amdgpu_waves_per_eu(4))) patch_kernel(const FreqP p) {
  __shared__ __attribute__((aligned(16))) unsigned char fw[2 * FBYTES];  // hi, then lo
  __shared__ __attribute__((aligned(16))) unsigned char iv[2 * IBYTES];
  for (int e = threadIdx.x; e < NCOEF * 16; e += 64 * PK_WAVES) {  // Fwd [80][64]: 16 groups of 4 per row
    const int r = e >> 4, k = (e & 15) * 4;
    const f32x4 f = *reinterpret_cast<const f32x4*>(p.fwd + r * 64 + k);
    put4_split(fw + r * FROWB + k * 2, fw + FBYTES + r * FROWB + k * 2, f);
  }
  stage_inv(iv, p.inv);
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform from here on
  const int lc = lane & 15, lg = lane >> 4;
  const int ph = (int)cdiv(p.h, 8), pw = (int)cdiv(p.w, 8);
  const int cblocks = (int)cdiv(p.c, 16);
  const int H = (int)p.h, W = (int)p.w;
  const int64_t C = p.c;
  constexpr int XES = (XDT == DT_BF16) ? 2 : 4;

  // Interior units (the whole 8 x 8 patch inside the image, all 16 channels present) address
  // everything from a wave-uniform base plus a per-lane offset fixed for the kernel, so the loads
  // and stores take scalar base addresses and no per-element vector arithmetic:
  //   x:     row 4 kb + lg of the patch, pixel s, channel lc: lane part lg sh + lc
  //   out:   patch row 2 ob + lg / 2, pixel 4 (lg % 2) + j, channel lc: lane part
  //          ((lg / 2) W + 4 (lg % 2)) C + lc (out and residual are dense NHWC)
  //   gains: coefficient 16 rb + 4 lg + j of channel lc: lane part 80 lc + 4 lg
  // (every byte offset from a unit's base below stays under 2^31)
  const bool fast_ok = (7 * p.sh + 7 * p.sw + 2 * C + 16) * XES < ((int64_t)1 << 31) &&
                       ((int64_t)8 * W * C + 16) * 4 < ((int64_t)1 << 31);
  const int xo_lane = fast_ok ? lg * (int)p.sh + lc : 0;
  const int oo_lane = fast_ok ? ((lg >> 1) * W + (lg & 1) * 4) * (int)C + lc : 0;
  const int go_lane = lc * NCOEF + lg * 4;
  const uint32_t xo_b = (uint32_t)xo_lane * XES, go_b = (uint32_t)go_lane * 4;

  struct UnitIn {
    f32x8 x[2], k[CORR ? 2 : 1];
    f32x4 g[CORR ? 1 : 5];
  };
  auto is_fast = [&](const PatchPos& q) __attribute__((always_inline)) {
    return fast_ok && q.py * 8 + 8 <= H && q.px * 8 + 8 <= W && (int64_t)q.cb * 16 + 16 <= C;
  };
  // a unit's inputs: this lane's 8 pixels of k-block kb (row 4 kb + lg of the patch, columns
  // 0..7), reflect padding at the bottom / right edge (torch F.pad mode="reflect"); and its
  // filter gains. The next unit's are loaded before the current one is computed, so their
  // memory latency overlaps the current unit's products and stores.
  // sh_l / sw_l / c_l: the strides, laundered per unit (below) so the scalar offsets derived from
  // them are recomputed per unit instead of held in scalar registers across the loop
  int sh_l = (int)p.sh, sw_l = (int)p.sw, c_l = (int)C, w_l = W;
  auto load_unit = [&](const PatchPos& q, UnitIn& in) __attribute__((always_inline)) {
    if (is_fast(q)) {
      // buffer loads: the unit's base in a scalar descriptor, the lane's offset in a VGPR fixed
      // for the kernel, the element's offset within the patch as a scalar
      const __amdgpu_buffer_rsrc_t xr = buf_rsrc(
          (const unsigned char*)p.x + (q.n * p.sn + (int64_t)(q.py * 8) * p.sh + (int64_t)(q.px * 8) * p.sw + q.cb * 16) * XES);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const int so = (kb * 4 * sh_l + s * sw_l) * XES;
          if constexpr (XDT == DT_BF16) {
            in.x[kb].v[s] = bf16_to_f32((unsigned short)__builtin_amdgcn_raw_buffer_load_b16(xr, (int)xo_b, so, 0));
            if constexpr (CORR)
              in.k[kb].v[s] = bf16_to_f32((unsigned short)__builtin_amdgcn_raw_buffer_load_b16(xr, (int)xo_b, so + c_l * 2, 0));
          } else {
            in.x[kb].v[s] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xr, (int)xo_b, so, 0));
            if constexpr (CORR)
              in.k[kb].v[s] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xr, (int)xo_b, so + c_l * 4, 0));
          }
        }
      if constexpr (!CORR) {
        const __amdgpu_buffer_rsrc_t gr = buf_rsrc(p.gain + (int64_t)q.cb * 16 * NCOEF);
#pragma unroll
        for (int rb = 0; rb < 5; ++rb)
          in.g[rb] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(gr, (int)go_b, rb * 64, 0));
      }
      return;
    }
    const int64_t ch = (int64_t)q.cb * 16 + lc;
    const bool cval = ch < C;
    const int64_t chl = cval ? ch : 0;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      int yy = q.py * 8 + kb * 4 + lg;
      if (yy >= H) yy = 2 * (H - 1) - yy;
      const int64_t rowoff = q.n * p.sn + (int64_t)yy * p.sh;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        int xx = q.px * 8 + s;
        if (xx >= W) xx = 2 * (W - 1) - xx;
        const int64_t o = rowoff + (int64_t)xx * p.sw;
        in.x[kb].v[s] = cval ? load1(p.x, XDT, o + chl) : 0.f;
        if constexpr (CORR) in.k[kb].v[s] = cval ? load1(p.x, XDT, o + C + chl) : 0.f;
      }
    }
    if constexpr (!CORR) {
#pragma unroll
      for (int rb = 0; rb < 5; ++rb)
        in.g[rb] = cval ? *reinterpret_cast<const f32x4*>(p.gain + chl * NCOEF + rb * 16 + lg * 4)
                        : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };

  // unit u = patch * cblocks + cb, patch = (n * ph + py) * pw + px; a wave steps by ustride units,
  // the position advanced with carries (no divisions in the loop)
  const int64_t ustride = (int64_t)gridDim.x * PK_WAVES;
  const int d_cb = (int)(ustride % cblocks);
  const int64_t d_patch = ustride / cblocks;
  const int d_px = (int)(d_patch % pw);
  const int64_t d_rows = d_patch / pw;
  const int d_py = (int)(d_rows % ph);
  const int64_t d_n = d_rows / ph;
  auto advance = [&](PatchPos& q) __attribute__((always_inline)) {
    q.cb += d_cb;
    int carry = q.cb >= cblocks;
    q.cb -= carry ? cblocks : 0;
    q.px += d_px + carry;
    carry = q.px >= pw;
    q.px -= carry ? pw : 0;
    q.py += d_py + carry;
    carry = q.py >= ph;
    q.py -= carry ? ph : 0;
    q.n += d_n + carry;
  };
  int64_t u = (int64_t)blockIdx.x * PK_WAVES + wave;
  PatchPos npos;
  {
    const int64_t patch = u / cblocks;
    npos.cb = (int)(u - patch * cblocks);
    const int64_t rows = patch / pw;
    npos.px = (int)(patch - rows * pw);
    npos.n = rows / ph;
    npos.py = (int)(rows - npos.n * ph);
  }
  UnitIn nxt;
  if (u < p.units) load_unit(npos, nxt);
  for (; u < p.units; u += ustride) {
    asm volatile("" ::: "memory");
    asm volatile("" : "+s"(sh_l), "+s"(sw_l), "+s"(c_l), "+s"(w_l));
    const UnitIn cur = nxt;
    const PatchPos cp = npos;
    advance(npos);
    if (u + ustride < p.units) load_unit(npos, nxt);

    bf16x8 xh[2], xl[2], kh[2], kl[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      split_bf16(cur.x[kb], xh[kb], xl[kb]);
      if constexpr (CORR) split_bf16(cur.k[kb], kh[kb], kl[kb]);
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
#pragma unroll
        for (int j = 0; j < 4; ++j) d1[rb][j] *= cur.g[rb][j];
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
    f32x4 y[4];
#pragma unroll
    for (int ob = 0; ob < 4; ++ob) {
      y[ob] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb2 = 0; kb2 < 3; ++kb2) {
        const int off = (ob * 16 + lc) * IROWB + (kb2 * 32 + lg * 8) * 2;
        const bf16x8 ih = lds8(iv + off), il = lds8(iv + IBYTES + off);
        y[ob] = mfma_bf16(ih, dh[kb2], y[ob]);
        y[ob] = mfma_bf16(ih, dl[kb2], y[ob]);
        y[ob] = mfma_bf16(il, dh[kb2], y[ob]);
      }
    }
    if (is_fast(cp)) {
      const int64_t ob0 = ((cp.n * H + cp.py * 8) * W + cp.px * 8) * C + cp.cb * 16;  // uniform
      // the 16 outputs of the lane, one residual / output dtype combination per unit (uniform)
      auto store_all = [&](auto res_c, auto out_c) __attribute__((always_inline)) {
        constexpr int RES = decltype(res_c)::value;  // 0 none, 2 bf16, 4 fp32
        constexpr int OES = decltype(out_c)::value;  // 2 bf16, 4 fp32
        const __amdgpu_buffer_rsrc_t orr = buf_rsrc((unsigned char*)p.out + ob0 * OES);
        const __amdgpu_buffer_rsrc_t rr = buf_rsrc(RES ? (const unsigned char*)p.res + ob0 * RES : (const unsigned char*)p.out);
        const int step_j = c_l, step_ob = 2 * w_l * c_l;  // element offsets within the patch
#pragma unroll
        for (int ob = 0; ob < 4; ++ob)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int eo = ob * step_ob + j * step_j;
            float v = y[ob][j];
            if constexpr (RES == 2) v += bf16_to_f32((unsigned short)__builtin_amdgcn_raw_buffer_load_b16(rr, oo_lane * 2, eo * 2, 0));
            if constexpr (RES == 4) v += __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rr, oo_lane * 4, eo * 4, 0));
            if constexpr (OES == 2) __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_bits(v), orr, oo_lane * 2, eo * 2, 0);
            else __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), orr, oo_lane * 4, eo * 4, 0);
          }
      };
      using I0 = std::integral_constant<int, 0>;
      using I2 = std::integral_constant<int, 2>;
      using I4 = std::integral_constant<int, 4>;
      const int rk = p.res ? (p.r_dt == DT_BF16 ? 2 : 4) : 0;
      if (p.o_dt == DT_BF16) {
        if (rk == 0) store_all(I0{}, I2{});
        else if (rk == 2) store_all(I2{}, I2{});
        else store_all(I4{}, I2{});
      } else {
        if (rk == 0) store_all(I0{}, I4{});
        else if (rk == 2) store_all(I2{}, I4{});
        else store_all(I4{}, I4{});
      }
    } else {
      const int64_t ch = (int64_t)cp.cb * 16 + lc;
      if (ch < C) {
#pragma unroll
        for (int ob = 0; ob < 4; ++ob) {
          const int pi0 = ob * 16 + lg * 4;  // pixels pi0 .. pi0 + 3: one patch row, 4 columns
          const int yy = cp.py * 8 + (pi0 >> 3);
          if (yy >= H) continue;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int xx = cp.px * 8 + (pi0 & 7) + j;
            if (xx >= W) continue;
            const int64_t o = ((cp.n * H + yy) * W + xx) * C + ch;  // out / residual contiguous
            float v = y[ob][j];
            if (p.res) v += load1(p.res, p.r_dt, o);
            store1(p.out, p.o_dt, o, v);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------- fused (LN) GEMM + patch filter
// out = patch_filter(prologue(x) . W + bias) (+ residual), the GEMM output never leaving the
// wave. Unit = (8x8 patch, CB blocks of 16 output channels), one wave:
//   GEMM  D[pb] (16 patch pixels 16 pb .. 16 pb + 15 as MFMA rows x the 16 channels) =
//         A[pixels][K] . W[K][channels] on 16x16x32 bf16 MFMAs; A rows are read straight from
//         the NHWC input (reflected coordinates past the bottom / right edge, which is the
//         reference's reflect padding of the GEMM output, since the GEMM is per pixel), with the
//         LayerNorm / RMS prologue applied in fp32 from the row values held in registers (the 4
//         lanes of a pixel row hold all K) and the normalised values entered as bf16 hi + lo
//         pairs (fp32 A too); with fp32 weights the GEMM runs on fp32 16x16x4 MFMAs instead.
//   lane (channel lc, group lg) then holds D[pb][j] = pixel 16 pb + 4 lg + j. The forward DFT
//   takes those registers as its B operand unchanged: its k slot (lg, i) of k-block kb stands
//   for pixel 32 kb + 16 (i / 4) + 4 lg + i % 4, and Fwd's columns are staged in that order.
//   Then gain, inverse, residual and store as patch_kernel. Each operator fragment read from LDS
//   and each A row read and normalised serves all CB channel blocks of the unit.
struct LpfP {
  const void* x;    // [batch, h, w, k] contiguous
  const void* wt;   // W^T [n][k]
  const float* bias;
  const float* fwd;
  const float* inv;
  const float* gain;  // [n][80]
  const void* res;
  void* out;          // [batch, h, w, n] contiguous
  int64_t batch, h, w, k, n;
  int64_t units;
  float eps;
  int r_dt, o_dt;
};

// W^T rows held in LDS (bf16 weights, N K 2 bytes at most this many): two workgroups per CU still fit
constexpr int LPF_WL_MAX = 30 * 1024;

// WL: the bf16 W^T [n][k] is copied into (dynamic) LDS once per workgroup and read from there.
template <int XDT, int LN, bool WS, int CB, int KS, bool WL>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) lpf_kernel(const LpfP p) {
  __shared__ __attribute__((aligned(16))) unsigned char fw[2 * FBYTES];  // Fwd hi, lo (columns permuted)
  __shared__ __attribute__((aligned(16))) unsigned char iv[2 * IBYTES];
  extern __shared__ __attribute__((aligned(16))) unsigned char wls[];    // W^T [n][k] bf16 (WL)
  if constexpr (WL) {
    const int nu = (int)(p.n * p.k / 8);  // 16-byte units
    for (int e = threadIdx.x; e < nu; e += 256)
      *reinterpret_cast<u32x4*>(wls + e * 16) = reinterpret_cast<const u32x4*>(p.wt)[e];
  }
  for (int e = threadIdx.x; e < NCOEF * 16; e += 256) {  // Fwd [80][64] in the GEMM's pixel order
    const int r = e >> 4, c4 = (e & 15) * 4;             // staged columns c4 .. c4 + 3
    const int kb = c4 >> 5, lgs = (c4 >> 3) & 3, i0 = c4 & 7;  // i0 = 0 or 4
    const int px0 = 32 * kb + 16 * (i0 >> 2) + 4 * lgs;  // 4 consecutive pixels
    const f32x4 f = *reinterpret_cast<const f32x4*>(p.fwd + r * 64 + px0);
    put4_split(fw + r * FROWB + c4 * 2, fw + FBYTES + r * FROWB + c4 * 2, f);
  }
  stage_inv(iv, p.inv);
  __syncthreads();

  constexpr bool AS = LN != 0 || XDT == DT_F32 || WS;  // A not entered as it stands
  constexpr int XES = XDT == DT_BF16 ? 2 : 4;
  constexpr int WES = WS ? 4 : 2;
  constexpr int MAXS = KS;                              // LN rows in registers: K <= 32 KS
  // patch-major order (LayerNorm rows normalised once per patch, held as hi + lo bf16 fragments
  // through all channel tiles) for bf16 weights and K <= 96
  constexpr bool PM = LN != 0 && !WS && KS <= 3;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lc = lane & 15, lg = lane >> 4;
  const int H = (int)p.h, W = (int)p.w, K = (int)p.k;
  const int ph = (int)cdiv(p.h, 8), pw = (int)cdiv(p.w, 8);
  const int ctiles = (int)cdiv(p.n, 16 * CB);  // channel tiles of CB 16-channel blocks
  // 8 bf16 weights of a W^T row at k0: from the LDS copy (WL) or global memory
  auto wload = [&](const unsigned char* row, int k0) __attribute__((always_inline)) -> bf16x8 {
    if constexpr (WL) {
      const int off = (int)(row - wls) + k0 * 2;
      return *reinterpret_cast<const bf16x8*>(wls + off);
    } else {
      return *reinterpret_cast<const bf16x8*>(row + (int64_t)k0 * 2);
    }
  };
  const int S = (int)cdiv(p.k, 32);            // 32-k steps
  const float invk = 1.0f / (float)K;

  // forward DFT, gains, inverse, + residual, store of one channel tile (GEMM outputs dd, + bias)
  // (lc, lg passed in: the patch-major loop hands over copies it re-derives per channel tile, so
  // the per-lane addresses built from them are not held across the loop)
  auto finish = [&](f32x4 (&dd)[CB][4], const int64_t (&chl)[CB], const bool (&cval)[CB], const int64_t n,
                    const int py, const int px, const int lc, const int lg) __attribute__((always_inline)) {
      // ---- forward DFT: B operand k-block kb = pixel blocks 2 kb (slots 0-3), 2 kb + 1 (4-7); each
      // operator fragment read from LDS once for the CB blocks
      bf16x8 xh[CB][2], xl[CB][2];
#pragma unroll
      for (int b = 0; b < CB; ++b)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          f32x8 xv;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            xv.v[j] = dd[b][2 * kb][j];
            xv.v[4 + j] = dd[b][2 * kb + 1][j];
          }
          split_bf16(xv, xh[b][kb], xl[b][kb]);
        }
      f32x4 d1[CB][5];
#pragma unroll
      for (int rb = 0; rb < 5; ++rb) {
#pragma unroll
        for (int b = 0; b < CB; ++b) d1[b][rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const int off = (rb * 16 + lc) * FROWB + (kb * 32 + lg * 8) * 2;
          const bf16x8 fh = lds8(fw + off), fl = lds8(fw + FBYTES + off);
#pragma unroll
          for (int b = 0; b < CB; ++b) {
            d1[b][rb] = mfma_bf16(fh, xh[b][kb], d1[b][rb]);
            d1[b][rb] = mfma_bf16(fh, xl[b][kb], d1[b][rb]);
            d1[b][rb] = mfma_bf16(fl, xh[b][kb], d1[b][rb]);
          }
        }
#pragma unroll
        for (int b = 0; b < CB; ++b) {
          const f32x4 g = cval[b] ? *reinterpret_cast<const f32x4*>(p.gain + chl[b] * NCOEF + rb * 16 + lg * 4)
                                  : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int j = 0; j < 4; ++j) d1[b][rb][j] *= g[j];
        }
      }
      bf16x8 dh[CB][3], dl[CB][3];
#pragma unroll
      for (int b = 0; b < CB; ++b)
#pragma unroll
        for (int kb2 = 0; kb2 < 3; ++kb2) {
          f32x8 dv;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            dv.v[j] = d1[b][2 * kb2][j];
            dv.v[4 + j] = (2 * kb2 + 1 < 5) ? d1[b][2 * kb2 + 1 < 5 ? 2 * kb2 + 1 : 0][j] : 0.f;
          }
          split_bf16(dv, dh[b][kb2], dl[b][kb2]);
        }
      // ---- inverse, residual, store
#pragma unroll
      for (int ob = 0; ob < 4; ++ob) {
        f32x4 y[CB];
#pragma unroll
        for (int b = 0; b < CB; ++b) y[b] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb2 = 0; kb2 < 3; ++kb2) {
          const int off = (ob * 16 + lc) * IROWB + (kb2 * 32 + lg * 8) * 2;
          const bf16x8 ih = lds8(iv + off), il = lds8(iv + IBYTES + off);
#pragma unroll
          for (int b = 0; b < CB; ++b) {
            y[b] = mfma_bf16(ih, dh[b][kb2], y[b]);
            y[b] = mfma_bf16(ih, dl[b][kb2], y[b]);
            y[b] = mfma_bf16(il, dh[b][kb2], y[b]);
          }
        }
        const int pi0 = ob * 16 + lg * 4;  // pixels pi0 .. pi0 + 3: one patch row, 4 columns
        const int yy = py * 8 + (pi0 >> 3);
        if (yy >= H) continue;
#pragma unroll
        for (int b = 0; b < CB; ++b) {
          if (!cval[b]) continue;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int xx = px * 8 + (pi0 & 7) + j;
            if (xx >= W) continue;
            const int64_t o = ((n * H + yy) * W + xx) * p.n + chl[b];
            float v = y[b][j];
            if (p.res) v += load1(p.res, p.r_dt, o);
            store1(p.out, p.o_dt, o, v);
          }
        }
      }
  };

  if constexpr (PM) {
    // one wave per patch: its 64 rows normalised once, held as MFMA A fragments (hi + lo bf16
    // pairs) through all channel tiles of the patch
    const int64_t npatch = p.batch * ph * pw;
    for (int64_t pt = (int64_t)blockIdx.x * 4 + wave; pt < npatch; pt += (int64_t)gridDim.x * 4) {
      asm volatile("" ::: "memory");
      const int64_t n = pt / ((int64_t)ph * pw);
      const int rem = (int)(pt - n * ph * pw);
      const int py = rem / pw, px = rem - (rem / pw) * pw;
      bf16x8 ah[4][KS], al[4][KS];
#pragma unroll
      for (int pb = 0; pb < 4; ++pb) {
        const int pp = pb * 16 + lc;  // this lane's A row: patch pixel pp
        int yy = py * 8 + (pp >> 3), xx = px * 8 + (pp & 7);
        if (yy >= H) yy = 2 * (H - 1) - yy;
        if (xx >= W) xx = 2 * (W - 1) - xx;
        const unsigned char* arow = (const unsigned char*)p.x + (((n * H + yy) * W + xx) * p.k) * XES;
        f32x8 a[KS];
        float s1 = 0.f;
#pragma unroll
        for (int st = 0; st < KS; ++st) {
          const int k0 = st * 32 + lg * 8;
          a[st] = (st < S && k0 < K) ? load8<XDT>(arow + (int64_t)k0 * XES) : zero8();
#pragma unroll
          for (int i = 0; i < 8; ++i) s1 += a[st].v[i];
        }
        const float mean = LN == 1 ? sum_col4(s1) * invk : 0.f;
        float s2 = 0.f;
#pragma unroll
        for (int st = 0; st < KS; ++st) {
          const bool kv = st < S && st * 32 + lg * 8 < K;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float d = kv ? a[st].v[i] - mean : 0.f;
            s2 += d * d;
          }
        }
        const float rstd = rsqrtf(sum_col4(s2) * invk + p.eps);
#pragma unroll
        for (int st = 0; st < KS; ++st) {
          const bool kv = st < S && st * 32 + lg * 8 < K;
          f32x8 v;
#pragma unroll
          for (int i = 0; i < 8; ++i) v.v[i] = kv ? (a[st].v[i] - mean) * rstd : 0.f;
          split_bf16(v, ah[pb][st], al[pb][st]);
        }
      }
#pragma unroll 1
      for (int ct = 0; ct < ctiles; ++ct) {
        asm volatile("" ::: "memory");
        int lc = lane & 15, lg = lane >> 4;
        asm volatile("" : "+v"(lc), "+v"(lg));
        int64_t chl[CB];
        bool cval[CB];
        const unsigned char* wrow[CB];
        f32x4 dd[CB][4];
#pragma unroll
        for (int b = 0; b < CB; ++b) {
          const int64_t ch = ((int64_t)ct * CB + b) * 16 + lc;
          cval[b] = ch < p.n;
          chl[b] = cval[b] ? ch : 0;
          wrow[b] = WL ? wls + chl[b] * p.k * 2 : (const unsigned char*)p.wt + chl[b] * p.k * WES;
          const float bv = (cval[b] && p.bias) ? p.bias[chl[b]] : 0.f;
#pragma unroll
          for (int pb = 0; pb < 4; ++pb) dd[b][pb] = f32x4{bv, bv, bv, bv};
        }
#pragma unroll
        for (int st = 0; st < KS; ++st) {
          if (st >= S) continue;
          const int k0 = st * 32 + lg * 8;
          const bool kv = k0 < K;
#pragma unroll
          for (int b = 0; b < CB; ++b) {
            const bf16x8 wv = (cval[b] && kv) ? wload(wrow[b], k0) : bf16x8{};
#pragma unroll
            for (int pb = 0; pb < 4; ++pb) {
              dd[b][pb] = mfma_bf16(ah[pb][st], wv, dd[b][pb]);
              dd[b][pb] = mfma_bf16(al[pb][st], wv, dd[b][pb]);
            }
          }
        }
        finish(dd, chl, cval, n, py, px, lc, lg);
      }
    }
  } else {
  for (int64_t u = (int64_t)blockIdx.x * 4 + wave; u < p.units; u += (int64_t)gridDim.x * 4) {
      asm volatile("" ::: "memory");
      const int ct = (int)(u % ctiles);
      const int64_t patch = u / ctiles;
      const int64_t n = patch / ((int64_t)ph * pw);
      const int rem = (int)(patch - n * ph * pw);
      const int py = rem / pw, px = rem - (rem / pw) * pw;
      int64_t chl[CB];
      bool cval[CB];
      const unsigned char* wrow[CB];
      float bias[CB];
#pragma unroll
      for (int b = 0; b < CB; ++b) {
        const int64_t ch = ((int64_t)ct * CB + b) * 16 + lc;
        cval[b] = ch < p.n;
        chl[b] = cval[b] ? ch : 0;
        wrow[b] = WL ? wls + chl[b] * p.k * 2 : (const unsigned char*)p.wt + chl[b] * p.k * WES;
        bias[b] = (cval[b] && p.bias) ? p.bias[chl[b]] : 0.f;
      }

      // ---- GEMM: dd[b][pb] = prologue(A) . W (channel block b), + bias; each A row is loaded and
      // normalised once for the CB blocks
      f32x4 dd[CB][4];
#pragma unroll
      for (int pb = 0; pb < 4; ++pb) {
        const int pp = pb * 16 + lc;  // this lane's A row: patch pixel pp
        int yy = py * 8 + (pp >> 3), xx = px * 8 + (pp & 7);
        if (yy >= H) yy = 2 * (H - 1) - yy;
        if (xx >= W) xx = 2 * (W - 1) - xx;
        const unsigned char* arow = (const unsigned char*)p.x + (((n * H + yy) * W + xx) * p.k) * XES;
#pragma unroll
        for (int b = 0; b < CB; ++b) dd[b][pb] = f32x4{bias[b], bias[b], bias[b], bias[b]};
        float mean = 0.f, rstd = 1.f;
        f32x8 a[LN != 0 ? MAXS : 1];
        if constexpr (LN != 0) {
          // the row in registers (K <= 256), exact two-pass statistics over the 4 lanes of the row
          float s1 = 0.f;
#pragma unroll
          for (int st = 0; st < MAXS; ++st) {
            const int k0 = st * 32 + lg * 8;
            a[st] = (st < S && k0 < K) ? load8<XDT>(arow + (int64_t)k0 * XES) : zero8();
#pragma unroll
            for (int i = 0; i < 8; ++i) s1 += a[st].v[i];
          }
          mean = LN == 1 ? sum_col4(s1) * invk : 0.f;
          float s2 = 0.f;
#pragma unroll
          for (int st = 0; st < MAXS; ++st) {
            const bool kv = st < S && st * 32 + lg * 8 < K;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const float d = kv ? a[st].v[i] - mean : 0.f;
              s2 += d * d;
            }
          }
          rstd = rsqrtf(sum_col4(s2) * invk + p.eps);
        }
        // LN rows: a constant trip count, fully unrolled (the row stays in registers); otherwise
        // a runtime loop over the steps (nothing indexed by the step)
        constexpr int NST = LN != 0 ? MAXS : 1;
#pragma unroll
        for (int st0 = 0; st0 < (LN != 0 ? NST : S); ++st0) {
          const int st = st0;
          if (LN != 0 && st >= S) continue;
          const int k0 = st * 32 + lg * 8;
          const bool kv = k0 < K;
          if constexpr (!AS) {  // bf16 rows and bf16 weights: one product
            const bf16x8 av = kv ? *reinterpret_cast<const bf16x8*>(arow + (int64_t)k0 * 2) : bf16x8{};
#pragma unroll
            for (int b = 0; b < CB; ++b) {
              const bf16x8 wv = (cval[b] && kv) ? wload(wrow[b], k0) : bf16x8{};
              dd[b][pb] = mfma_bf16(av, wv, dd[b][pb]);
            }
          } else {
            f32x8 v;
            if constexpr (LN != 0) {
#pragma unroll
              for (int i = 0; i < 8; ++i) v.v[i] = kv ? (a[st0 < NST ? st0 : 0].v[i] - mean) * rstd : 0.f;
            } else {
              v = kv ? load8<XDT>(arow + (int64_t)k0 * XES) : zero8();
            }
            if constexpr (WS) {  // fp32 weights: fp32 MFMAs, slot i = instruction i's k
#pragma unroll
              for (int b = 0; b < CB; ++b) {
                const f32x8 wv = (cval[b] && kv) ? load8<DT_F32>(wrow[b] + (int64_t)k0 * 4) : zero8();
#pragma unroll
                for (int i = 0; i < 8; ++i) dd[b][pb] = mfma_f32(v.v[i], wv.v[i], dd[b][pb]);
              }
            } else {  // bf16 weights: A as hi + lo pairs
              bf16x8 ah, al;
              split_bf16(v, ah, al);
#pragma unroll
              for (int b = 0; b < CB; ++b) {
                const bf16x8 wv = (cval[b] && kv) ? wload(wrow[b], k0) : bf16x8{};
                dd[b][pb] = mfma_bf16(ah, wv, dd[b][pb]);
                dd[b][pb] = mfma_bf16(al, wv, dd[b][pb]);
              }
            }
          }
        }
      }

      finish(dd, chl, cval, n, py, px, lc, lg);
    }
  }
}

static int launch_patch(FreqP& p, hipStream_t s, const char* what) {
  p.small_offsets = (7 * p.sh + 7 * p.sw + 2 * p.c) < ((int64_t)1 << 31) && p.sh < ((int64_t)1 << 31) &&
                    p.sw < ((int64_t)1 << 31);
  const int64_t patches = p.batch * cdiv(p.h, 8) * cdiv(p.w, 8);
  p.units = patches * cdiv(p.c, 16);
  // persistent: 2 resident workgroups per CU (the LDS operator copies), so each stages the
  // matrices once for many units
  int64_t blocks = cdiv(p.units, PK_WAVES);
  if (blocks > 2LL * device_cus()) blocks = 2LL * device_cus();
  const dim3 g((unsigned)blocks);
  if (p.corr) {
    note_kernel("patch_kernel corr=1");
    if (p.x_dt == DT_BF16) hipLaunchKernelGGL((patch_kernel<DT_BF16, true>), g, dim3(64 * PK_WAVES), 0, s, p);
    else hipLaunchKernelGGL((patch_kernel<DT_F32, true>), g, dim3(64 * PK_WAVES), 0, s, p);
  } else {
    note_kernel("patch_kernel corr=0");
    if (p.x_dt == DT_BF16) hipLaunchKernelGGL((patch_kernel<DT_BF16, false>), g, dim3(64 * PK_WAVES), 0, s, p);
    else hipLaunchKernelGGL((patch_kernel<DT_F32, false>), g, dim3(64 * PK_WAVES), 0, s, p);
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

// dynamic LDS beyond the default 64 KiB per workgroup (static operators + the W^T copy)
static void lpf_allow_lds(const void* fn) {
  (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, LPF_WL_MAX);
}

extern "C" int clarus_hip_linear_patch_filter(const void* x, int32_t x_dtype, const void* wt, int32_t w_dtype,
                                              const float* bias, int32_t ln, float ln_eps, const float* fwd,
                                              const float* inv, const float* gain, const void* res, int32_t r_dtype,
                                              void* out, int32_t o_dtype, int64_t batch, int64_t h, int64_t w,
                                              int64_t k, int64_t n, void* stream) {
  clear_error();
  CLARUS_REQUIRE(x && wt && fwd && inv && gain && out, "linear_patch_filter: null operand");
  CLARUS_REQUIRE(batch > 0 && h > 0 && w > 0 && k > 0 && n > 0, "linear_patch_filter: bad sizes");
  CLARUS_REQUIRE((x_dtype == DT_F32 || x_dtype == DT_BF16) && (w_dtype == DT_F32 || w_dtype == DT_BF16) &&
                     (o_dtype == DT_F32 || o_dtype == DT_BF16), "linear_patch_filter: bad dtype");
  CLARUS_REQUIRE(ln >= 0 && ln <= 2, "linear_patch_filter: ln is 0 (none), 1 (LayerNorm) or 2 (RMS)");
  CLARUS_REQUIRE(k % 8 == 0 && (ln == 0 || k <= 256), "linear_patch_filter: K=%lld must be a multiple of 8 (and <= 256 "
                 "with a LayerNorm / RMS prologue)", (long long)k);
  CLARUS_REQUIRE(h >= 9 && w >= 9, "linear_patch_filter: reflect padding to a multiple of 8 needs h, w >= 9");
  CLARUS_REQUIRE(aligned(x, 16) && aligned(wt, 16) && aligned(gain, 16) && aligned(fwd, 16) && aligned(inv, 16),
                 "linear_patch_filter: 16-byte alignment");
  CLARUS_REQUIRE(batch * h * w * (k > n ? k : n) < ((int64_t)1 << 62), "linear_patch_filter: too large");
  if (res) CLARUS_REQUIRE(r_dtype == DT_F32 || r_dtype == DT_BF16, "linear_patch_filter: bad residual dtype");
  LpfP p{};
  p.x = x; p.wt = wt; p.bias = bias; p.fwd = fwd; p.inv = inv; p.gain = gain; p.res = res; p.out = out;
  p.batch = batch; p.h = h; p.w = w; p.k = k; p.n = n;
  p.eps = ln_eps; p.r_dt = r_dtype; p.o_dt = o_dtype;
  // channel tile: 2 16-channel blocks of one patch per wave (operator fragments and A rows reused
  // twice; 3 blocks hold ~230 VGPRs, one wave per SIMD, and ran 1.19 against 0.96 ms at the
  // FFTformer level-0 DFFN shape). With a LayerNorm / RMS prologue the row is held in KS 32-k
  // steps, the fewest that cover K. bf16 W^T of at most LPF_WL_MAX bytes is read from LDS.
  const int cb = 2;
  const bool wl = w_dtype == DT_BF16 && n * k * 2 <= LPF_WL_MAX;
  const size_t wl_bytes = wl ? (size_t)(n * k * 2) : 0;
  const int steps = (int)cdiv(k, 32);
  const int ks = steps <= 2 ? 2 : steps <= 3 ? 3 : steps <= 4 ? 4 : steps <= 6 ? 6 : 8;
  p.units = batch * cdiv(h, 8) * cdiv(w, 8) * cdiv(n, 16 * cb);
  // persistent: 2 resident workgroups per CU (the two-block tile holds ~170 VGPRs: 2 waves per
  // SIMD; the operators and a W^T copy take ~76 KiB of LDS)
  int64_t blocks = cdiv(p.units, 4);
  if (blocks > 2LL * device_cus()) blocks = 2LL * device_cus();
  const dim3 g((unsigned)blocks);
  hipStream_t s = (hipStream_t)stream;
  // instantiated: LayerNorm / RMS prologues for bf16 activations with bf16 weights and fp32 with
  // fp32 (the two backends); no prologue for every dtype pair (the rows pass feeds bf16 rows to
  // fp32 weights)
  const bool same = (x_dtype == DT_BF16) == (w_dtype == DT_BF16);
  CLARUS_REQUIRE(ln == 0 || same, "linear_patch_filter: a LayerNorm / RMS prologue needs activations and weights "
                 "of one dtype");
  note_kernel("lpf_kernel ln=%d ws=%d cb=%d ks=%d wl=%d", ln, w_dtype == DT_F32, cb, ln ? ks : 0, (int)wl);
  // WL copies only for W^T within LPF_WL_MAX (K <= 48 at N = 6K): instantiated for KS <= 2
#define CLARUS_LPF_CB(XDT, LNV, WSV, KSV)                                                                  \
  do {                                                                                                     \
    if (!WSV && wl && KSV <= 2) {                                                                          \
      lpf_allow_lds(reinterpret_cast<const void*>(&lpf_kernel<XDT, LNV, WSV, 2, KSV, !WSV && KSV <= 2>));  \
      hipLaunchKernelGGL((lpf_kernel<XDT, LNV, WSV, 2, KSV, !WSV && KSV <= 2>), g, dim3(256), wl_bytes, s, \
                         p);                                                                               \
    } else {                                                                                               \
      hipLaunchKernelGGL((lpf_kernel<XDT, LNV, WSV, 2, KSV, false>), g, dim3(256), 0, s, p);               \
    }                                                                                                      \
  } while (0)
#define CLARUS_LPF_KS(XDT, LNV, WSV)                   \
  do {                                                 \
    switch (ks) {                                      \
      case 2: CLARUS_LPF_CB(XDT, LNV, WSV, 2); break;  \
      case 3: CLARUS_LPF_CB(XDT, LNV, WSV, 3); break;  \
      case 4: CLARUS_LPF_CB(XDT, LNV, WSV, 4); break;  \
      case 6: CLARUS_LPF_CB(XDT, LNV, WSV, 6); break;  \
      default: CLARUS_LPF_CB(XDT, LNV, WSV, 8); break; \
    }                                                  \
  } while (0)
  if (ln == 0) {
    if (x_dtype == DT_BF16) {
      if (w_dtype == DT_F32) CLARUS_LPF_CB(DT_BF16, 0, true, 1);
      else CLARUS_LPF_CB(DT_BF16, 0, false, 1);
    } else {
      if (w_dtype == DT_F32) CLARUS_LPF_CB(DT_F32, 0, true, 1);
      else CLARUS_LPF_CB(DT_F32, 0, false, 1);
    }
  } else if (x_dtype == DT_BF16) {
    if (ln == 1) CLARUS_LPF_KS(DT_BF16, 1, false);
    else CLARUS_LPF_KS(DT_BF16, 2, false);
  } else {
    if (ln == 1) CLARUS_LPF_KS(DT_F32, 1, true);
    else CLARUS_LPF_KS(DT_F32, 2, true);
  }
#undef CLARUS_LPF_KS
#undef CLARUS_LPF_CB
  return check_launch("linear_patch_filter");
}
