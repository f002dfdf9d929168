// Fused NHWC GEMM / implicit-GEMM convolution for gfx950.
//
// out[p, n] = epilogue( sum_k prologue(A)[p, k] * W[k, n] )
//
// Work decomposition ("pixel-major"): the MFMA computes D[channel][pixel] = W^T . A^T, so a
// lane's accumulators are 4 consecutive output channels of one pixel.
//   * a workgroup (4 waves) owns TN = 16 * NB output channels (x2 rows of W^T with SimpleGate)
//     and walks over pixel tiles of TP = 64 * PB pixels (persistent: tile = blockIdx.x,
//     blockIdx.x + gridDim.x, ...);
//   * each wave owns 16 * PB pixels of the tile and all TN channels;
//   * W^T (K contiguous) is staged into LDS in chunks of KC; the rows are placed so that the
//     4 * NB channels a lane accumulates are contiguous in memory (vector stores);
//   * activations are loaded straight from global memory in MFMA operand layout: one lane
//     reads 8 consecutive k of one pixel (16 B of bf16), so the NHWC row is the operand and
//     any per-element prologue (LayerNorm, local-mean multiply, LN*m) is applied in fp32 on
//     the way into the MFMA. No LDS round trip for the big operand.
// Operand modes (OPM):
//   0  bf16 A (raw, no prologue) x bf16 W : one bf16 MFMA per k-step (products exact in fp32)
//   1  fp32-valued A (fp32 input or any prologue) x bf16 W: A = hi + lo in bf16, two MFMAs
//   2  fp32 A x fp32 W: fp32 MFMA (16x16x4), eight per 32-k step
// A addressing (AM): 0 NHWC rows with stride lda (+ prologue), 1 2x2 stride-2 space-to-depth,
//   2 implicit 3x3 convolution (zero padding, optional nearest-x2 input).
#pragma once

#include "common.hpp"

namespace clarus {

enum : int { PRO_NONE = 0, PRO_LN = 1, PRO_MUL = 2, PRO_RMS = 3, PRO_LNMUL = 5 };
enum : int { AM_ROWS = 0, AM_S2D = 1, AM_CONV3 = 2 };
enum : int { CM_ROWS = 0, CM_SHUFFLE = 1, CM_NCHW = 2 };
enum : int { ACT_NONE = 0, ACT_GELU = 1, ACT_LRELU = 2 };
enum : int { OPM_BF16 = 0, OPM_SPLIT = 1, OPM_F32 = 2 };

struct GemmP {
  const void* a;
  const void* wt;
  void* c;
  const float* bias;
  const float* scale;
  const void* res;
  const void* small;
  const void* m2;
  const float* lnw;
  const float* lnb;
  int64_t m, n, k;
  int64_t lda, ldc, ldr, ldm2;
  int64_t a_bs, w_bs, c_bs, r_bs, s_bs, m2_bs;
  int64_t ptiles;
  int c_dt, r_dt, s_dt, m2_dt;
  int h, w;          // AM_S2D / CM_SHUFFLE: input size; AM_CONV3: input size; PRO_MUL: image size
  int oh, ow, pt, pl;
  int cin;           // AM_S2D / AM_CONV3 input channels
  int up2;           // AM_CONV3: nearest x2 input
  int pro, c_mode, act, m2_act;
  int has_bias, has_scale, has_res, vec_out, vec_res;
  float ln_eps, out_scale, slope;
};

template <int TA>
__device__ __forceinline__ constexpr int esz() { return TA == DT_BF16 ? 2 : 4; }

// ---------------------------------------------------------------------------------------
template <int NB, int PB, bool GATE, int OPM, int TA, int AM, int KC>
__global__ void __launch_bounds__(256) gemm_kernel(const GemmP p) {
  constexpr int G = GATE ? 2 : 1;
  constexpr int TN = NB * 16;
  constexpr int TP = PB * 64;
  constexpr bool WF32 = (OPM == OPM_F32);
  constexpr int WES = WF32 ? 4 : 2;            // bytes per staged W element
  constexpr int ROW = KC + (WF32 ? 4 : 8);     // LDS row length (elements), +16 B pad
  constexpr int UNIT = 16 / WES;               // elements per 16-byte copy unit
  constexpr int NKS = KC / 32;                 // k-steps per chunk
  __shared__ __attribute__((aligned(16))) unsigned char lds[G * TN * ROW * WES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lc = lane & 15;  // pixel within a 16-pixel block (MFMA column)
  const int lg = lane >> 4;  // lane group: selects k within a step and channels in the run
  const int64_t n0 = (int64_t)blockIdx.y * TN;
  const int64_t bz = blockIdx.z;

  const unsigned char* A = (const unsigned char*)p.a + bz * p.a_bs * esz<TA>();
  const unsigned char* Wt = (const unsigned char*)p.wt + bz * p.w_bs * WES;
  const int64_t K = p.k;
  const int nchunks = (int)cdiv(K, KC);

  // ---- stage W^T rows [n0, n0 + TN) (and the gate half) for k in [k0, k0 + KC) into LDS
  auto stage_w = [&](int64_t k0) {
    constexpr int UPR = KC / UNIT;  // units per row
    for (int u = tid; u < G * TN * UPR; u += 256) {
      const int r = u / UPR;
      const int cu = u - r * UPR;
      const int half = r / TN;
      const int rr = r - half * TN;
      const int nb = rr >> 4;
      const int ri = rr & 15;
      const int64_t ch = n0 + (ri >> 2) * (4 * NB) + nb * 4 + (ri & 3);
      const int64_t kk = k0 + (int64_t)cu * UNIT;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (ch < p.n && kk < K) {
        const int64_t row = half * p.n + ch;
        v = *reinterpret_cast<const u32x4*>(Wt + (row * K + kk) * WES);
      }
      *reinterpret_cast<u32x4*>(lds + ((size_t)r * ROW + cu * UNIT) * WES) = v;
    }
  };

  if (nchunks == 1) {
    stage_w(0);
    __syncthreads();
  }

  const int hw_out = (AM == AM_CONV3) ? (p.h << p.up2) * (p.w << p.up2)
                     : (AM == AM_S2D) ? (p.h >> 1) * (p.w >> 1) : 0;
  const int wo = (AM == AM_CONV3) ? (p.w << p.up2) : (AM == AM_S2D) ? (p.w >> 1) : 0;
  const int ho = (AM == AM_CONV3) ? (p.h << p.up2) : (AM == AM_S2D) ? (p.h >> 1) : 0;

  for (int64_t tile = blockIdx.x; tile < p.ptiles; tile += gridDim.x) {
    const int64_t pbase = tile * TP + wave * (PB * 16);

    // per pixel-block geometry of this lane's pixel
    int64_t pix[PB];
    bool pval[PB];
    int img[PB], py[PB], px[PB];
    const unsigned char* arow[PB];
#pragma unroll
    for (int b = 0; b < PB; ++b) {
      pix[b] = pbase + b * 16 + lc;
      pval[b] = pix[b] < p.m;
      const int64_t q = pval[b] ? pix[b] : 0;
      if constexpr (AM == AM_ROWS) {
        arow[b] = A + q * p.lda * esz<TA>();
        img[b] = py[b] = px[b] = 0;
      } else {
        img[b] = (int)(q / hw_out);
        const int rr = (int)(q - (int64_t)img[b] * hw_out);
        py[b] = rr / wo;
        px[b] = rr - py[b] * wo;
        if constexpr (AM == AM_S2D)
          arow[b] = A + ((((int64_t)img[b] * p.h + 2 * py[b]) * p.w + 2 * px[b]) * p.cin) * esz<TA>();
        else
          arow[b] = A;
      }
    }

    // ---- row statistics for the LayerNorm prologues (exact two-pass, fp32)
    float mean[PB], rstd[PB];
#pragma unroll
    for (int b = 0; b < PB; ++b) { mean[b] = 0.f; rstd[b] = 1.f; }
    if constexpr (AM == AM_ROWS) {
      if (p.pro == PRO_LN || p.pro == PRO_LNMUL || p.pro == PRO_RMS) {
        const float invk = 1.0f / (float)K;
#pragma unroll
        for (int b = 0; b < PB; ++b) {
          float s = 0.f;
          if (p.pro != PRO_RMS) {
            if (pval[b])
              for (int64_t k = lg * 8; k < K; k += 32) {
                f32x8 a = load8<TA>(arow[b] + k * esz<TA>());
#pragma unroll
                for (int i = 0; i < 8; ++i) s += a.v[i];
              }
            s = sum_col4(s);
            mean[b] = s * invk;
          }
          float ss = 0.f;
          if (pval[b])
            for (int64_t k = lg * 8; k < K; k += 32) {
              f32x8 a = load8<TA>(arow[b] + k * esz<TA>());
#pragma unroll
              for (int i = 0; i < 8; ++i) {
                const float d = a.v[i] - mean[b];
                ss += d * d;
              }
            }
          ss = sum_col4(ss);
          rstd[b] = rsqrtf(ss * invk + p.ln_eps);
        }
      }
    }

    f32x4 acc[PB][NB];
    f32x4 acc2[GATE ? PB : 1][GATE ? NB : 1];
#pragma unroll
    for (int b = 0; b < PB; ++b)
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        acc[b][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        if constexpr (GATE) acc2[b][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      }

    for (int ch = 0; ch < nchunks; ++ch) {
      const int64_t k0 = (int64_t)ch * KC;
      if (nchunks > 1) {
        __syncthreads();
        stage_w(k0);
        __syncthreads();
      }
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const int64_t kb = k0 + ks * 32;
        if (kb >= K) break;  // uniform
        const int64_t k = kb + lg * 8;
        const bool kval = k < K;

        // ---- activation fragments (8 consecutive k of this lane's pixel)
        f32x8 xf[PB];
        bf16x8 xb[PB];
#pragma unroll
        for (int b = 0; b < PB; ++b) {
          bool ok = pval[b] && kval;
          const unsigned char* src = arow[b];
          if constexpr (AM == AM_ROWS) {
            src += k * esz<TA>();
          } else if constexpr (AM == AM_S2D) {
            const int q = (int)(k / p.cin);
            const int c = (int)(k - (int64_t)q * p.cin);
            src += ((int64_t)((q >> 1) * p.w + (q & 1)) * p.cin + c) * esz<TA>();
          } else {  // AM_CONV3
            const int tap = (int)(k / p.cin);
            const int c = (int)(k - (int64_t)tap * p.cin);
            int yy = py[b] + tap / 3 - 1;
            int xx = px[b] + tap % 3 - 1;
            ok = ok && yy >= 0 && yy < ho && xx >= 0 && xx < wo;
            yy >>= p.up2;
            xx >>= p.up2;
            src = A + ((((int64_t)img[b] * p.h + yy) * p.w + xx) * p.lda + c) * esz<TA>();
          }
          if constexpr (OPM == OPM_BF16) {
            u32x4 raw = {0u, 0u, 0u, 0u};
            if (ok) raw = *reinterpret_cast<const u32x4*>(src);
            xb[b] = __builtin_bit_cast(bf16x8, raw);
          } else {
            f32x8 a = ok ? load8<TA>(src) : zero8();
            if constexpr (AM == AM_ROWS) {
              if (ok && p.pro != PRO_NONE) {
                if (p.pro == PRO_LN) {
#pragma unroll
                  for (int i = 0; i < 8; ++i) a.v[i] = (a.v[i] - mean[b]) * rstd[b];
                } else if (p.pro == PRO_RMS) {
#pragma unroll
                  for (int i = 0; i < 8; ++i) a.v[i] = a.v[i] * rstd[b];
                } else if (p.pro == PRO_MUL) {
                  const int64_t q = pix[b];
                  const int hwi = p.h * p.w;
                  const int64_t im = q / hwi;
                  const int rr = (int)(q - im * hwi);
                  int sy = rr / p.w - p.pt;
                  int sx = rr % p.w - p.pl;
                  sy = sy < 0 ? 0 : (sy > p.oh - 1 ? p.oh - 1 : sy);
                  sx = sx < 0 ? 0 : (sx > p.ow - 1 ? p.ow - 1 : sx);
                  const int64_t srow = (im * p.oh + sy) * p.ow + sx;
                  const unsigned char* sp = (const unsigned char*)p.small;
                  f32x8 s = (p.s_dt == DT_BF16)
                                ? load8<DT_BF16>(sp + (bz * p.s_bs + srow * K + k) * 2)
                                : load8<DT_F32>(sp + (bz * p.s_bs + srow * K + k) * 4);
#pragma unroll
                  for (int i = 0; i < 8; ++i) a.v[i] *= s.v[i];
                } else {  // PRO_LNMUL
                  const unsigned char* mp = (const unsigned char*)p.m2;
                  const int64_t mo = bz * p.m2_bs + pix[b] * p.ldm2 + k;
                  f32x8 mv = (p.m2_dt == DT_BF16) ? load8<DT_BF16>(mp + mo * 2)
                                                  : load8<DT_F32>(mp + mo * 4);
                  f32x8 lw = load8<DT_F32>(p.lnw + k);
                  f32x8 lb = load8<DT_F32>(p.lnb + k);
#pragma unroll
                  for (int i = 0; i < 8; ++i) {
                    float mm = mv.v[i];
                    if (p.m2_act == ACT_GELU) mm = gelu_erf(mm);
                    const float t = (a.v[i] - mean[b]) * rstd[b];
                    a.v[i] = (t * lw.v[i] + lb.v[i]) * mm;
                  }
                }
              }
            }
            xf[b] = a;
          }
        }

        // ---- W fragments from LDS and the products
#pragma unroll
        for (int j = 0; j < NB; ++j) {
#pragma unroll
          for (int hf = 0; hf < G; ++hf) {
            const size_t off = ((size_t)(hf * TN + j * 16 + lc) * ROW + ks * 32 + lg * 8) * WES;
            if constexpr (WF32) {
              f32x8 wv;
              f32x4 w0 = *reinterpret_cast<const f32x4*>(lds + off);
              f32x4 w1 = *reinterpret_cast<const f32x4*>(lds + off + 16);
#pragma unroll
              for (int i = 0; i < 4; ++i) { wv.v[i] = w0[i]; wv.v[4 + i] = w1[i]; }
#pragma unroll
              for (int b = 0; b < PB; ++b) {
                f32x4 t = hf ? acc2[GATE ? b : 0][GATE ? j : 0] : acc[b][j];
#pragma unroll
                for (int i = 0; i < 8; ++i) t = mfma_f32(wv.v[i], xf[b].v[i], t);
                if (hf) acc2[GATE ? b : 0][GATE ? j : 0] = t; else acc[b][j] = t;
              }
            } else {
              const bf16x8 wv = *reinterpret_cast<const bf16x8*>(lds + off);
#pragma unroll
              for (int b = 0; b < PB; ++b) {
                f32x4 t = hf ? acc2[GATE ? b : 0][GATE ? j : 0] : acc[b][j];
                if constexpr (OPM == OPM_BF16) {
                  t = mfma_bf16(wv, xb[b], t);
                } else {
                  bf16x8 hi, lo;
                  split_bf16(xf[b], hi, lo);
                  t = mfma_bf16(wv, hi, t);
                  t = mfma_bf16(wv, lo, t);
                }
                if (hf) acc2[GATE ? b : 0][GATE ? j : 0] = t; else acc[b][j] = t;
              }
            }
          }
        }
      }
    }

    // ---- epilogue: + bias -> gate -> act -> * scale -> * out_scale -> + residual -> store
    const int64_t run0 = n0 + lg * (4 * NB);
#pragma unroll
    for (int b = 0; b < PB; ++b) {
      if (!pval[b]) continue;
      const int64_t q = pix[b];
      int64_t obase = 0, rbase = 0;  // element offsets of channel 0 of this pixel
      int64_t cstride = 1;           // element distance between consecutive channels
      int64_t qstride = 0;           // CM_SHUFFLE: extra offset per quadrant
      int64_t cq = 0;                // CM_SHUFFLE: channels per quadrant
      if (p.c_mode == CM_ROWS) {
        obase = bz * p.c_bs + q * p.ldc;
        rbase = bz * p.r_bs + q * p.ldr;
      } else if (p.c_mode == CM_SHUFFLE) {
        const int64_t hwi = (int64_t)p.h * p.w;
        const int64_t im = q / hwi;
        const int rr = (int)(q - im * hwi);
        const int y = rr / p.w, x = rr - (rr / p.w) * p.w;
        cq = p.n >> 2;
        obase = (((im * 2 * p.h + 2 * y) * 2 * p.w) + 2 * x) * cq;
        rbase = obase;
        qstride = 0;
      } else {  // CM_NCHW (conv output size ho x wo)
        const int64_t hwo = (int64_t)ho * wo;
        const int64_t im = q / hwo;
        const int64_t rr = q - im * hwo;
        obase = im * p.n * hwo + rr;
        rbase = obase;
        cstride = hwo;
      }
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int64_t c0 = run0 + j * 4;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t c = c0 + i;
          const bool cv = c < p.n;
          float x = acc[b][j][i];
          if (p.has_bias && cv) x += p.bias[c];
          if constexpr (GATE) {
            float x2 = acc2[b][j][i];
            if (p.has_bias && cv) x2 += p.bias[p.n + c];
            x = x * x2;
          }
          if (p.act == ACT_GELU) x = gelu_erf(x);
          else if (p.act == ACT_LRELU) x = x >= 0.f ? x : x * p.slope;
          if (p.has_scale && cv) x = x * p.scale[c];
          if (p.out_scale != 1.0f) x = x * p.out_scale;
          v[i] = x;
        }
        // addresses of the quad's first channel
        int64_t oo, ro;
        if (p.c_mode == CM_SHUFFLE) {
          const int64_t qd = c0 / cq;
          const int64_t cc = c0 - qd * cq;
          const int64_t add = ((qd >> 1) * 2 * p.w + (qd & 1)) * cq + cc;
          oo = obase + add;
          ro = rbase + add;
        } else {
          oo = obase + c0 * cstride;
          ro = rbase + c0 * cstride;
        }
        const bool full = (c0 + 3 < p.n);
        if (p.has_res) {
          if (full && p.vec_res && cstride == 1) {
            if (p.r_dt == DT_BF16) {
              u32x2 r = *reinterpret_cast<const u32x2*>((const unsigned short*)p.res + ro);
              v[0] += __uint_as_float(r[0] << 16);
              v[1] += __uint_as_float(r[0] & 0xffff0000u);
              v[2] += __uint_as_float(r[1] << 16);
              v[3] += __uint_as_float(r[1] & 0xffff0000u);
            } else {
              f32x4 r = *reinterpret_cast<const f32x4*>((const float*)p.res + ro);
#pragma unroll
              for (int i = 0; i < 4; ++i) v[i] += r[i];
            }
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (c0 + i < p.n) v[i] += load1(p.res, p.r_dt, ro + i * cstride);
          }
        }
        if (full && p.vec_out && cstride == 1) {
          if (p.c_dt == DT_BF16) {
            u32x2 o;
            o[0] = (unsigned)f32_to_bf16_bits(v[0]) | ((unsigned)f32_to_bf16_bits(v[1]) << 16);
            o[1] = (unsigned)f32_to_bf16_bits(v[2]) | ((unsigned)f32_to_bf16_bits(v[3]) << 16);
            *reinterpret_cast<u32x2*>((unsigned short*)p.c + oo) = o;
          } else {
            *reinterpret_cast<f32x4*>((float*)p.c + oo) = f32x4{v[0], v[1], v[2], v[3]};
          }
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (c0 + i < p.n) store1(p.c, p.c_dt, oo + i * cstride, v[i]);
        }
      }
    }
  }
}

}  // namespace clarus
