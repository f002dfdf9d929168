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
//   * W^T (K contiguous) is staged into LDS in chunks of KC (double-buffered when K > KC; kept
//     resident for the whole persistent loop when K <= KC); the rows are placed so that the
//     4 * NB channels a lane accumulates are contiguous in memory (16-byte vector stores);
//   * activations are loaded straight from global memory in MFMA operand layout: one lane
//     reads 8 consecutive k of one pixel (16 B of bf16), so the NHWC row is the operand and
//     any per-element prologue (LayerNorm, local-mean multiply, LN*m) is applied in fp32 on
//     the way into the MFMA. A whole chunk of fragments is loaded before any is used, and
//     LayerNorm statistics come from those registers when K fits one chunk.
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
// operand modes: bf16 products; fp32 A (or a prologue output) as hi + lo bf16 pairs; fp32
// products; a prologue output rounded once to bf16 (ring streaming kernel)
enum : int { OPM_BF16 = 0, OPM_SPLIT = 1, OPM_F32 = 2, OPM_ROUND = 3 };

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
  const float* stats;  // per-row (mean, rstd) from the statistics pass, or null
  int64_t m, n, k;
  int64_t lda, ldc, ldr, ldm2;
  int64_t a_bs, w_bs, c_bs, r_bs;
  int64_t ptiles;
  int c_dt, r_dt, s_dt, m2_dt;
  int h, w;          // AM_S2D / CM_SHUFFLE / AM_CONV3: input size; PRO_MUL: image size
  int oh, ow, pt, pl;
  int cin;           // AM_S2D / AM_CONV3 input channels
  int s2d;           // gemm_mfma32_kernel: A rows are 2x2 stride-2 windows of an NHWC image (h, w, cin)
  int up2;           // AM_CONV3: nearest x2 input
  int pro, c_mode, act, m2_act;
  int has_res;
  int vec_out, vec_res;  // widest aligned vector access of the output / residual: 2 = 16 B, 1 = 8 B, 0 = scalar
  float ln_eps, out_scale, slope;
};

template <int TA>
__device__ __forceinline__ constexpr int esz() { return TA == DT_BF16 ? 2 : 4; }

// raw activation fragment: 8 consecutive k of one pixel
template <int TA> struct RawFrag;
template <> struct RawFrag<DT_BF16> { u32x4 q; };
template <> struct RawFrag<DT_F32> { f32x4 a, b; };

template <int TA>
__device__ __forceinline__ RawFrag<TA> raw_zero() {
  RawFrag<TA> r;
  if constexpr (TA == DT_BF16) r.q = u32x4{0u, 0u, 0u, 0u};
  else r.a = r.b = f32x4{0.f, 0.f, 0.f, 0.f};
  return r;
}

template <int TA>
__device__ __forceinline__ RawFrag<TA> raw_load(const unsigned char* p) {
  RawFrag<TA> r;
  if constexpr (TA == DT_BF16) r.q = *reinterpret_cast<const u32x4*>(p);
  else { r.a = reinterpret_cast<const f32x4*>(p)[0]; r.b = reinterpret_cast<const f32x4*>(p)[1]; }
  return r;
}

template <int TA>
__device__ __forceinline__ f32x8 raw_f32(const RawFrag<TA>& r) {
  f32x8 o;
  if constexpr (TA == DT_BF16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o.v[2 * i] = __uint_as_float(r.q[i] << 16);
      o.v[2 * i + 1] = __uint_as_float(r.q[i] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) { o.v[i] = r.a[i]; o.v[4 + i] = r.b[i]; }
  }
  return o;
}

// LDS bytes of one W^T buffer (G * TN rows of KC elements + a 16-byte pad) and of the
// epilogue vectors (bias of both gate halves and scale), per instantiation
__host__ __device__ constexpr int gemm_wbuf_bytes(int nb, bool gate, int opm, int kc) {
  return (gate ? 2 : 1) * nb * 16 * (kc + (opm == 2 ? 4 : 8)) * (opm == 2 ? 4 : 2);
}
__host__ __device__ constexpr int gemm_epi_bytes(int nb) { return 3 * nb * 16 * 4; }

__device__ __forceinline__ void wait_vmem_all() {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); expcnt / lgkmcnt untouched
}

// ---------------------------------------------------------------------------------------
template <int NB, int PB, bool GATE, int OPM, int TA, int AM, int KC>
__global__ void __launch_bounds__(256) gemm_kernel(const GemmP p) {
  constexpr int G = GATE ? 2 : 1;
  constexpr int TN = NB * 16;
  constexpr int TP = PB * 64;
  constexpr int RUN = 4 * NB;                  // contiguous channels per lane
  constexpr bool WF32 = (OPM == OPM_F32);
  constexpr int WES = WF32 ? 4 : 2;            // bytes per staged W element
  constexpr int ROW = KC + (WF32 ? 4 : 8);     // LDS row length (elements), +16 B pad
  constexpr int ROWB = ROW * WES;
  constexpr int UNIT = 16 / WES;               // elements per 16-byte copy unit
  constexpr int NKS = KC / 32;                 // k-steps per chunk
  constexpr int BUF = gemm_wbuf_bytes(NB, GATE, OPM, KC);
  static_assert(BUF == G * TN * ROWB, "W buffer layout");
  // dynamic LDS: [epilogue vectors][W buffer 0][W buffer 1 (K > KC only)]
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  float* epi = reinterpret_cast<float*>(lds);  // [G * TN] bias, then [TN] scale (tile order)
  unsigned char* wlds = lds + gemm_epi_bytes(NB);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lc = lane & 15;  // pixel within a 16-pixel block (MFMA column)
  const int lg = lane >> 4;  // lane group: selects k within a step and the channel run
  const int64_t n0 = (int64_t)blockIdx.y * TN;
  const int64_t bz = blockIdx.z;
  const int64_t run0 = n0 + lg * RUN;

  const unsigned char* A = (const unsigned char*)p.a + bz * p.a_bs * esz<TA>();
  const unsigned char* Wt = (const unsigned char*)p.wt + bz * p.w_bs * WES;
  const int64_t K = p.k;
  const int nchunks = (int)cdiv(K, KC);

  // ---- epilogue vectors of the tile's channels, in channel order
  for (int i = tid; i < (G + 1) * TN; i += 256) {
    const int part = i / TN;  // 0 bias, 1 gate-half bias (G == 2), last: scale
    const int64_t c = n0 + (i - part * TN);
    float v;
    if (part < G) v = (p.bias && c < p.n) ? p.bias[part * p.n + c] : 0.f;
    else v = ((p.scale && c < p.n) ? p.scale[c] : 1.f) * p.out_scale;
    epi[i] = v;
  }
  const bool full_n = (n0 + TN) <= p.n;

  // ---- W^T chunk [k0, k0 + KC) of rows [n0, n0 + TN) (+ gate half) -> LDS buffer, by direct
  // global->LDS 16-byte copies: lane i of a wave writes bytes [base + 16 i, base + 16 i + 16).
  // Tile row r holds the channel whose accumulator lands in lane run order; sources past the
  // last channel / K are clamped into the tensor (finite values that only meet zero operands or
  // feed unstored rows), the 16-byte row pad takes any valid source.
  auto w_dma = [&](int64_t k0, int buf) {
    unsigned char* dst = wlds + buf * BUF;
    for (int base = wave * 1024; base < BUF; base += 4 * 1024) {
      const int pos = base + lane * 16;
      if (pos < BUF) {
        const int r = pos / ROWB;
        int cb = pos - r * ROWB;
        if (cb >= KC * WES) cb = 0;
        const int half = r / TN;
        const int rr = r - half * TN;
        int64_t ch = n0 + ((rr & 15) >> 2) * RUN + (rr >> 4) * 4 + (rr & 3);
        if (ch > p.n - 1) ch = p.n - 1;
        int64_t kk = k0 + cb / WES;
        if (kk > K - UNIT) kk = K - UNIT;
        const unsigned char* src = Wt + ((half * p.n + ch) * K + kk) * WES;
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                         (__attribute__((address_space(3))) void*)(dst + base), 16, 0, 0);
      }
    }
  };

  if (nchunks == 1) w_dma(0, 0);
  wait_vmem_all();
  __syncthreads();

  const int ho = (AM == AM_CONV3) ? (p.h << p.up2) : (AM == AM_S2D) ? (p.h >> 1) : 1;
  const int wo = (AM == AM_CONV3) ? (p.w << p.up2) : (AM == AM_S2D) ? (p.w >> 1) : 1;
  const int hw_out = ho * wo;
  const bool stats = (AM == AM_ROWS) && (p.pro == PRO_LN || p.pro == PRO_LNMUL || p.pro == PRO_RMS);

  for (int64_t tile = blockIdx.x; tile < p.ptiles; tile += gridDim.x) {
    const int64_t pbase = tile * TP + wave * (PB * 16);

    // ---- this lane's pixel in each 16-pixel block
    int64_t pix[PB];
    bool pval[PB];
    int img[PB], py[PB], px[PB];
    const unsigned char* arow[PB];
#pragma unroll
    for (int b = 0; b < PB; ++b) {
      pix[b] = pbase + b * 16 + lc;
      pval[b] = pix[b] < p.m;
      const int64_t q = pval[b] ? pix[b] : 0;
      img[b] = py[b] = px[b] = 0;
      if constexpr (AM == AM_ROWS) {
        arow[b] = A + q * p.lda * esz<TA>();
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

    // address of the fragment (pixel block b, k = kb + 8 lg); ok is false for padding /
    // out-of-image taps. kb is uniform: one scalar division per k-step, then a per-lane wrap.
    auto frag_src = [&](int b, int64_t kb, bool& ok) -> const unsigned char* {
      const int64_t k = kb + lg * 8;
      ok = pval[b] && k < K;
      if constexpr (AM == AM_ROWS) {
        return arow[b] + k * esz<TA>();
      } else {
        int t = (int)(kb / p.cin);
        int c = (int)(kb - (int64_t)t * p.cin) + lg * 8;
        while (c >= p.cin) { c -= p.cin; ++t; }
        if constexpr (AM == AM_S2D) {
          return arow[b] + ((int64_t)((t >> 1) * p.w + (t & 1)) * p.cin + c) * esz<TA>();
        } else {
          const int t3 = t / 3;
          int yy = py[b] + t3 - 1;
          int xx = px[b] + (t - 3 * t3) - 1;
          ok = ok && yy >= 0 && yy < ho && xx >= 0 && xx < wo;
          yy >>= p.up2;
          xx >>= p.up2;
          return A + ((((int64_t)img[b] * p.h + yy) * p.w + xx) * p.lda + c) * esz<TA>();
        }
      }
    };

    // element offsets of this pixel's rows in the mul map / the LN*m multiplier
    int64_t xrow[PB];
#pragma unroll
    for (int b = 0; b < PB; ++b) {
      xrow[b] = 0;
      if constexpr (AM == AM_ROWS) {
        if (p.pro == PRO_MUL) {
          const int hwi = p.h * p.w;
          const int64_t q = pval[b] ? pix[b] : 0;
          const int64_t im = q / hwi;
          const int rr = (int)(q - im * hwi);
          const int yq = rr / p.w;
          int sy = yq - p.pt, sx = rr - yq * p.w - p.pl;
          sy = sy < 0 ? 0 : (sy > p.oh - 1 ? p.oh - 1 : sy);
          sx = sx < 0 ? 0 : (sx > p.ow - 1 ? p.ow - 1 : sx);
          xrow[b] = ((im * p.oh + sy) * p.ow + sx) * K;
        } else if (p.pro == PRO_LNMUL) {
          xrow[b] = (pval[b] ? pix[b] : 0) * p.ldm2;
        }
      }
    }

    // ---- LayerNorm statistics (two-pass) when K spans several chunks: read the rows first
    float mean[PB], rstd[PB];
#pragma unroll
    for (int b = 0; b < PB; ++b) { mean[b] = 0.f; rstd[b] = 1.f; }
    if (stats && nchunks > 1 && p.stats) {  // precomputed by the statistics pass
#pragma unroll
      for (int b = 0; b < PB; ++b) {
        const f32x2 st = pval[b] ? *reinterpret_cast<const f32x2*>(p.stats + 2 * pix[b]) : f32x2{0.f, 1.f};
        mean[b] = st[0];
        rstd[b] = st[1];
      }
    } else if (stats && nchunks > 1) {
      const float invk = 1.0f / (float)K;
#pragma unroll
      for (int b = 0; b < PB; ++b) {
        float s = 0.f, ss = 0.f;
        if (p.pro != PRO_RMS) {
          if (pval[b])
            for (int64_t k = lg * 8; k < K; k += 32) {
              const f32x8 a = raw_f32<TA>(raw_load<TA>(arow[b] + k * esz<TA>()));
#pragma unroll
              for (int i = 0; i < 8; ++i) s += a.v[i];
            }
          mean[b] = sum_col4(s) * invk;
        }
        if (pval[b])
          for (int64_t k = lg * 8; k < K; k += 32) {
            const f32x8 a = raw_f32<TA>(raw_load<TA>(arow[b] + k * esz<TA>()));
#pragma unroll
            for (int i = 0; i < 8; ++i) { const float d = a.v[i] - mean[b]; ss += d * d; }
          }
        rstd[b] = rsqrtf(sum_col4(ss) * invk + p.ln_eps);
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

    if (nchunks > 1) {  // prime the W pipeline for this tile
      __syncthreads();   // every wave is done with the previous tile's buffers
      w_dma(0, 0);
    }

    for (int chunk = 0; chunk < nchunks; ++chunk) {
      const int64_t k0 = (int64_t)chunk * KC;
      const int buf = (nchunks > 1) ? (chunk & 1) : 0;
      const bool more = chunk + 1 < nchunks;
      if (nchunks > 1) {  // chunk's W landed (this thread's copies, then everyone's)
        wait_vmem_all();
        __syncthreads();
        if (more) w_dma(k0 + KC, buf ^ 1);  // next chunk streams in while this one computes
      }

      // ---- all activation fragments of this chunk
      RawFrag<TA> raw[NKS][PB];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
        for (int b = 0; b < PB; ++b) {
          bool ok;
          const unsigned char* src = frag_src(b, k0 + ks * 32, ok);
          raw[ks][b] = ok ? raw_load<TA>(src) : raw_zero<TA>();
        }

      if (stats && nchunks == 1) {  // whole row in registers: exact two-pass statistics
        const float invk = 1.0f / (float)K;
#pragma unroll
        for (int b = 0; b < PB; ++b) {
          float s = 0.f;
          if (p.pro != PRO_RMS) {
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
              const f32x8 a = raw_f32<TA>(raw[ks][b]);
#pragma unroll
              for (int i = 0; i < 8; ++i) s += a.v[i];
            }
            mean[b] = sum_col4(s) * invk;
          }
          float ss = 0.f;
#pragma unroll
          for (int ks = 0; ks < NKS; ++ks) {
            if (k0 + ks * 32 + lg * 8 >= K) continue;
            const f32x8 a = raw_f32<TA>(raw[ks][b]);
#pragma unroll
            for (int i = 0; i < 8; ++i) { const float d = a.v[i] - mean[b]; ss += d * d; }
          }
          rstd[b] = rsqrtf(sum_col4(ss) * invk + p.ln_eps);
        }
      }

#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const int64_t kb = k0 + ks * 32;
        if (kb >= K) break;  // uniform
        const int64_t k = kb + lg * 8;

        // ---- operand fragments (prologue in fp32)
        f32x8 xf[PB];
        bf16x8 xb[PB];
#pragma unroll
        for (int b = 0; b < PB; ++b) {
          if constexpr (OPM == OPM_BF16) {
            xb[b] = __builtin_bit_cast(bf16x8, raw[ks][b].q);
          } else {
            f32x8 a = raw_f32<TA>(raw[ks][b]);
            if constexpr (AM == AM_ROWS) {
              const bool ok = pval[b] && k < K;
              if (p.pro == PRO_LN) {
#pragma unroll
                for (int i = 0; i < 8; ++i) a.v[i] = (a.v[i] - mean[b]) * rstd[b];
              } else if (p.pro == PRO_RMS) {
#pragma unroll
                for (int i = 0; i < 8; ++i) a.v[i] = a.v[i] * rstd[b];
              } else if (p.pro == PRO_MUL && ok) {
                const int64_t so = xrow[b] + k;
                const f32x8 s = (p.s_dt == DT_BF16)
                                    ? load8<DT_BF16>((const unsigned char*)p.small + so * 2)
                                    : load8<DT_F32>((const unsigned char*)p.small + so * 4);
#pragma unroll
                for (int i = 0; i < 8; ++i) a.v[i] *= s.v[i];
              } else if (p.pro == PRO_LNMUL && ok) {
                const int64_t mo = xrow[b] + k;
                const f32x8 mv = (p.m2_dt == DT_BF16) ? load8<DT_BF16>((const unsigned char*)p.m2 + mo * 2)
                                                      : load8<DT_F32>((const unsigned char*)p.m2 + mo * 4);
                const f32x8 lw = load8<DT_F32>(p.lnw + k);
                const f32x8 lb = load8<DT_F32>(p.lnb + k);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                  const float mm = (p.m2_act == ACT_GELU) ? gelu_erf(mv.v[i]) : mv.v[i];
                  const float t = (a.v[i] - mean[b]) * rstd[b];
                  a.v[i] = (t * lw.v[i] + lb.v[i]) * mm;
                }
              }
              if (!ok) a = zero8();
            }
            xf[b] = a;
          }
        }

        // ---- W fragments from LDS and the products
#pragma unroll
        for (int j = 0; j < NB; ++j) {
#pragma unroll
          for (int hf = 0; hf < G; ++hf) {
            const size_t off = buf * BUF + (size_t)(hf * TN + j * 16 + lc) * ROWB + (ks * 32 + lg * 8) * WES;
            if constexpr (WF32) {
              f32x8 wv;
              const f32x4 w0 = *reinterpret_cast<const f32x4*>(wlds + off);
              const f32x4 w1 = *reinterpret_cast<const f32x4*>(wlds + off + 16);
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
              const bf16x8 wv = *reinterpret_cast<const bf16x8*>(wlds + off);
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

    // ---- epilogue: + bias -> gate -> act -> * scale (* out_scale) -> + residual -> store
#pragma unroll
    for (int b = 0; b < PB; ++b) {
      if (!pval[b]) continue;
      const int64_t q = pix[b];
      float v[RUN];
      const int e0 = lg * RUN;  // this lane's run within the tile
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const f32x4 b1 = *reinterpret_cast<const f32x4*>(epi + e0 + j * 4);
        f32x4 b2 = b1;
        if constexpr (GATE) b2 = *reinterpret_cast<const f32x4*>(epi + TN + e0 + j * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float x = acc[b][j][i] + b1[i];
          if constexpr (GATE) x = x * (acc2[b][j][i] + b2[i]);
          v[j * 4 + i] = x;
        }
      }
      if (p.act == ACT_GELU) {
#pragma unroll
        for (int i = 0; i < RUN; ++i) v[i] = gelu_erf(v[i]);
      } else if (p.act == ACT_LRELU) {
#pragma unroll
        for (int i = 0; i < RUN; ++i) v[i] = v[i] >= 0.f ? v[i] : v[i] * p.slope;
      }
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const f32x4 sc = *reinterpret_cast<const f32x4*>(epi + G * TN + e0 + j * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[j * 4 + i] *= sc[i];
      }

      // element offsets of channel run0 of this pixel (and the per-channel stride)
      int64_t oo, ro, cs = 1;
      if (AM == AM_CONV3 && p.c_mode == CM_NCHW) {
        const int64_t im = q / hw_out;
        const int64_t rr = q - im * hw_out;
        oo = (im * p.n + run0) * hw_out + rr;
        ro = oo;
        cs = hw_out;
      } else if (p.c_mode == CM_SHUFFLE) {
        const int64_t hwi = (int64_t)p.h * p.w;
        const int64_t im = q / hwi;
        const int rr = (int)(q - im * hwi);
        const int y = rr / p.w, x = rr - (rr / p.w) * p.w;
        const int64_t cq = p.n >> 2;
        const int64_t qd = run0 / cq, cc = run0 - qd * cq;
        oo = ((im * 2 * p.h + 2 * y + (qd >> 1)) * 2 * p.w + 2 * x + (qd & 1)) * cq + cc;
        ro = oo;
      } else {
        oo = bz * p.c_bs + q * p.ldc + run0;
        ro = bz * p.r_bs + q * p.ldr + run0;
      }
      const bool vec = full_n && cs == 1;
      if (p.has_res) {
        if (vec && p.vec_res) {
          if (p.r_dt == DT_BF16) {
            const unsigned short* rp = (const unsigned short*)p.res + ro;
#pragma unroll
            for (int j = 0; j < RUN / 4; ++j) {
              const u32x2 r = *reinterpret_cast<const u32x2*>(rp + 4 * j);
              v[4 * j] += __uint_as_float(r[0] << 16);
              v[4 * j + 1] += __uint_as_float(r[0] & 0xffff0000u);
              v[4 * j + 2] += __uint_as_float(r[1] << 16);
              v[4 * j + 3] += __uint_as_float(r[1] & 0xffff0000u);
            }
          } else {
            const float* rp = (const float*)p.res + ro;
#pragma unroll
            for (int j = 0; j < RUN / 4; ++j) {
              const f32x4 r = *reinterpret_cast<const f32x4*>(rp + 4 * j);
#pragma unroll
              for (int i = 0; i < 4; ++i) v[4 * j + i] += r[i];
            }
          }
        } else {
#pragma unroll
          for (int i = 0; i < RUN; ++i)
            if (run0 + i < p.n) v[i] += load1(p.res, p.r_dt, ro + i * cs);
        }
      }
      if (vec && p.vec_out) {
        if (p.c_dt == DT_BF16) {
          unsigned short* op = (unsigned short*)p.c + oo;
          u32x2 o[RUN / 4];
#pragma unroll
          for (int j = 0; j < RUN / 4; ++j) {
            o[j][0] = (unsigned)f32_to_bf16_bits(v[4 * j]) | ((unsigned)f32_to_bf16_bits(v[4 * j + 1]) << 16);
            o[j][1] = (unsigned)f32_to_bf16_bits(v[4 * j + 2]) | ((unsigned)f32_to_bf16_bits(v[4 * j + 3]) << 16);
          }
          if (RUN >= 8 && p.vec_out == 2) {
#pragma unroll
            for (int j = 0; j + 1 < RUN / 4; j += 2)
              *reinterpret_cast<u32x4*>(op + 4 * j) = u32x4{o[j][0], o[j][1], o[j + 1][0], o[j + 1][1]};
          } else {
#pragma unroll
            for (int j = 0; j < RUN / 4; ++j) *reinterpret_cast<u32x2*>(op + 4 * j) = o[j];
          }
        } else {
          float* op = (float*)p.c + oo;
#pragma unroll
          for (int j = 0; j < RUN / 4; ++j)
            *reinterpret_cast<f32x4*>(op + 4 * j) = f32x4{v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]};
        }
      } else {
#pragma unroll
        for (int i = 0; i < RUN; ++i)
          if (run0 + i < p.n) store1(p.c, p.c_dt, oo + i * cs, v[i]);
      }
    }
  }
}

}  // namespace clarus
