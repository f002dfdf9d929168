// Pipelined LDS-tiled fused GEMM for NHWC rows with long K (the MFMA-bound NAFNet levels 3-4,
// K = 512 / 1024), gfx950.
//
// Same math and output mapping as gemm_kernel (D[channel][pixel] = W^T . A^T on MFMA, a lane
// accumulates runs of consecutive output channels of one pixel), different data movement:
//   * a workgroup computes a 128-pixel x 128-W^T-row tile (128 output channels, or 64 with
//     SimpleGate: both halves of each channel sit in the same lane); its 4 waves split it 2 x 2,
//     each wave 64 pixels x 64 rows = 4 x 4 MFMA blocks per 32-k step;
//   * per K chunk (KC), W^T rows and A rows are staged through registers: each thread loads
//     its 16-byte W units and 8-k A fragments, applies the prologue to A (LN / RMS with
//     precomputed row statistics, local-mean multiply, LN * m) and the bf16 hi / lo split once,
//     and writes both to LDS, so no wave repeats that work (register staging rather than direct
//     global->LDS copies: the compiler then needs no memory wait before the LDS reads of the
//     chunk being computed while the next chunk's loads are in flight);
//   * the (tile, chunk) steps of a workgroup form one flat pipeline with two LDS stages: the
//     global loads of step s + 1 are in flight while step s computes, with a single barrier per
//     step, also across tile boundaries;
//   * tiles are dealt out XCD-aware: the tiles of one XCD form a contiguous range with the
//     column tiles of a pixel tile adjacent, so the A rows are fetched from HBM into that XCD's
//     L2 once and reused by the other column tiles.
#pragma once

#include "gemm_kernel.hpp"

namespace clarus {

constexpr int LT_P = 128;  // pixels per tile
constexpr int LT_R = 128;  // W^T rows per tile

__host__ __device__ constexpr int lt_rowb(int kc) { return (kc + 8) * 2; }  // bf16 row + 16 B pad
__host__ __device__ constexpr int lt_wbuf(int kc) { return LT_R * lt_rowb(kc); }
__host__ __device__ constexpr int lt_abuf(int kc, int opm) { return (opm == OPM_SPLIT ? 2 : 1) * LT_P * lt_rowb(kc); }
__host__ __device__ constexpr int lt_lds_bytes(int kc, int opm) { return 2 * (lt_wbuf(kc) + lt_abuf(kc, opm)); }

// residual add + store of one lane's run of RUN output channels (v in fp32, channel run0 ..)
template <int RUN>
__device__ __forceinline__ void store_run(const GemmP& p, float (&v)[RUN], int64_t oo, int64_t ro, int64_t run0,
                                          bool vec) {
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
        if (run0 + i < p.n) v[i] += load1(p.res, p.r_dt, ro + i);
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
      if (run0 + i < p.n) store1(p.c, p.c_dt, oo + i, v[i]);
  }
}

template <int OPM, int TA, bool GATE, bool X2, int KC>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) gemm_lds_kernel(const GemmP p) {
  static_assert(OPM == OPM_BF16 || OPM == OPM_SPLIT, "bf16 weights only");
  static_assert(KC % 32 == 0 && (LT_P * KC / 8) % 256 == 0, "chunk shape");
  constexpr int G = GATE ? 2 : 1;
  constexpr int TNO = LT_R / G;        // output channels per tile
  constexpr int WCH = TNO / 2;         // output channels per wave
  constexpr int RUN = WCH / 4;         // contiguous channels per lane (16, gate 8)
  constexpr int ROWB = lt_rowb(KC);
  constexpr int WBUF = lt_wbuf(KC);
  constexpr int ABUF = lt_abuf(KC, OPM);
  constexpr int STAGE = WBUF + ABUF;
  constexpr int NKS = KC / 32;
  constexpr int FQ = KC / 8;                 // 8-k fragments per pixel row of a chunk
  constexpr int FPT = LT_P * FQ / 256;       // A fragments (and W^T units) staged per thread per chunk
  extern __shared__ __attribute__((aligned(16))) unsigned char stages[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lc = lane & 15, lg = lane >> 4;
  const int wp = wave & 1, wn = wave >> 1;
  const int64_t K = p.k;
  const int nch = (int)cdiv(K, KC);
  const int ntn = (int)cdiv(p.n, TNO);
  const int T = (int)p.ptiles * ntn;  // the host checks that this fits 31 bits
  const unsigned char* A = (const unsigned char*)p.a;
  const unsigned char* Wt = (const unsigned char*)p.wt;

  // XCD-aware deal: workgroup b runs on XCD b % 8 and takes tiles xcd * span + b / 8 + j * per
  const int xcd = blockIdx.x & 7;
  const int per = gridDim.x >> 3;
  const int span = (T + 7) >> 3;
  const int t0 = xcd * span + (blockIdx.x >> 3);
  const int t_end = (xcd + 1) * span < T ? (xcd + 1) * span : T;
  const int ntiles = t0 < t_end ? (t_end - t0 + per - 1) / per : 0;
  const int nsteps = ntiles * nch;

  // ---- staging: this thread's A fragments f = tid + 256 i (pixel f / FQ, k = k0 + 8 (f % FQ))
  // and W^T units u = tid + 256 i (tile row u / FQ, same k), loaded into registers one step
  // ahead, transformed and written to LDS after the current step's products.
  RawFrag<TA> ra[FPT];
  u32x4 rw[FPT];
  RawFrag<DT_F32> rx[X2 ? FPT : 1];
  const unsigned char* a_src[FPT];  // per tile: row + unit offset at k = 0
  const unsigned char* w_src[FPT];
  const unsigned char* x_src[X2 ? FPT : 1];
  f32x2 rst[FPT];
  bool pv[FPT];
  int is_tile = 0, is_chunk = 0;
  int64_t is_k0 = 0;

  auto set_issue_tile = [&]() __attribute__((always_inline)) {
    const int t = t0 + is_tile * per;
    const int pt = t / ntn, nt = t - pt * ntn;
#pragma unroll
    for (int i = 0; i < FPT; ++i) {
      const int f = tid + 256 * i;
      const int64_t q = (int64_t)pt * LT_P + f / FQ;
      pv[i] = q < p.m;
      const int64_t qc = pv[i] ? q : p.m - 1;
      a_src[i] = A + (qc * p.lda + (f % FQ) * 8) * esz<TA>();
      rst[i] = f32x2{0.f, 1.f};
      if constexpr (OPM == OPM_SPLIT)
        if (p.stats) rst[i] = *reinterpret_cast<const f32x2*>(p.stats + 2 * qc);
      if constexpr (X2) {
        int64_t xo;
        if (p.pro == PRO_MUL) {
          const int hwi = p.h * p.w;
          const int64_t im = qc / hwi;
          const int rr = (int)(qc - im * hwi);
          const int yq = rr / p.w;
          int sy = yq - p.pt, sx = rr - yq * p.w - p.pl;
          sy = sy < 0 ? 0 : (sy > p.oh - 1 ? p.oh - 1 : sy);
          sx = sx < 0 ? 0 : (sx > p.ow - 1 ? p.ow - 1 : sx);
          xo = ((im * p.oh + sy) * p.ow + sx) * K;
        } else {
          xo = qc * p.ldm2;
        }
        const int dt = (p.pro == PRO_MUL) ? p.s_dt : p.m2_dt;
        const unsigned char* b = (const unsigned char*)((p.pro == PRO_MUL) ? p.small : p.m2);
        x_src[i] = b + (xo + (f % FQ) * 8) * (dt == DT_BF16 ? 2 : 4);
      }
      // W^T: tile row r holds the channel that makes a lane's accumulators a contiguous run;
      // rows past the last channel are clamped into the tensor (their outputs are not stored)
      const int r = f / FQ;
      int half, ch;
      if constexpr (GATE) {
        half = r >> 6;
        const int rl = r & 63, w2 = rl >> 5, r2 = rl & 31;
        ch = w2 * 32 + ((r2 & 15) >> 2) * 8 + (r2 >> 4) * 4 + (r2 & 3);
      } else {
        half = 0;
        const int w2 = r >> 6, r2 = r & 63;
        ch = w2 * 64 + ((r2 & 15) >> 2) * 16 + (r2 >> 4) * 4 + (r2 & 3);
      }
      int64_t c = (int64_t)nt * TNO + ch;
      if (c > p.n - 1) c = p.n - 1;
      w_src[i] = Wt + ((half * p.n + c) * K + (f % FQ) * 8) * 2;
    }
  };

  auto issue = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < FPT; ++i) {
      const int f = tid + 256 * i;
      const int64_t k = is_k0 + (f % FQ) * 8;
      const bool kok = k < K;
      // W^T past K: clamped to the last 8 k (they meet zero A)
      const int64_t wk = kok ? is_k0 : (K - 8 - (f % FQ) * 8);
      rw[i] = *reinterpret_cast<const u32x4*>(w_src[i] + wk * 2);
      ra[i] = (pv[i] && kok) ? raw_load<TA>(a_src[i] + is_k0 * esz<TA>()) : raw_zero<TA>();
      if constexpr (X2) {
        RawFrag<DT_F32> v;
        v.a = v.b = f32x4{0.f, 0.f, 0.f, 0.f};
        if (pv[i] && kok) {
          const int dt = (p.pro == PRO_MUL) ? p.s_dt : p.m2_dt;
          const f32x8 t8 = dt == DT_BF16 ? load8<DT_BF16>(x_src[i] + is_k0 * 2) : load8<DT_F32>(x_src[i] + is_k0 * 4);
          v.a = f32x4{t8.v[0], t8.v[1], t8.v[2], t8.v[3]};
          v.b = f32x4{t8.v[4], t8.v[5], t8.v[6], t8.v[7]};
        }
        rx[i] = v;
      }
    }
  };
  auto advance_issue = [&]() __attribute__((always_inline)) {
    if (++is_chunk == nch) {
      is_chunk = 0;
      is_k0 = 0;
      ++is_tile;
      if (is_tile < ntiles) set_issue_tile();
    } else {
      is_k0 += KC;
    }
  };

  // prologue + split of the staged registers into LDS stage sb (k0 of the staged chunk)
  auto commit = [&](int sb, int64_t k0) __attribute__((always_inline)) {
    unsigned char* wbuf = stages + sb * STAGE;
    unsigned char* abuf = wbuf + WBUF;
#pragma unroll
    for (int i = 0; i < FPT; ++i) {
      const int f = tid + 256 * i;
      const int off = (f / FQ) * ROWB + (f % FQ) * 16;
      *reinterpret_cast<u32x4*>(wbuf + off) = rw[i];
      if constexpr (OPM == OPM_BF16) {
        *reinterpret_cast<u32x4*>(abuf + off) = ra[i].q;
      } else {
        f32x8 a = raw_f32<TA>(ra[i]);
        const int64_t k = k0 + (f % FQ) * 8;
        const float mean = rst[i][0], rstd = rst[i][1];
        if (p.pro == PRO_LN) {
#pragma unroll
          for (int e = 0; e < 8; ++e) a.v[e] = (a.v[e] - mean) * rstd;
        } else if (p.pro == PRO_RMS) {
#pragma unroll
          for (int e = 0; e < 8; ++e) a.v[e] = a.v[e] * rstd;
        }
        if constexpr (X2) {
          const f32x8 m = raw_f32<DT_F32>(rx[i]);
          if (p.pro == PRO_MUL) {
#pragma unroll
            for (int e = 0; e < 8; ++e) a.v[e] *= m.v[e];
          } else {  // PRO_LNMUL
            const bool kok = k < K;
            const f32x8 lw = kok ? load8<DT_F32>(p.lnw + k) : zero8();
            const f32x8 lb = kok ? load8<DT_F32>(p.lnb + k) : zero8();
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float mm = (p.m2_act == ACT_GELU) ? gelu_erf(m.v[e]) : m.v[e];
              a.v[e] = (((a.v[e] - mean) * rstd) * lw.v[e] + lb.v[e]) * mm;
            }
          }
        }
        if (!(pv[i] && k < K)) a = zero8();
        bf16x8 hi, lo;
        split_bf16(a, hi, lo);
        *reinterpret_cast<bf16x8*>(abuf + off) = hi;
        *reinterpret_cast<bf16x8*>(abuf + LT_P * ROWB + off) = lo;
      }
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  // W^T row of the wave's MFMA row block rb (gate: blocks 0, 1 first half, 2, 3 second half)
  auto wrow = [&](int rb) { return GATE ? ((rb >> 1) * 64 + wn * 32 + (rb & 1) * 16) : (wn * 64 + rb * 16); };

  if (nsteps == 0) return;
  set_issue_tile();
  issue();
  commit(0, 0);
  advance_issue();
  __syncthreads();
  int s = 0;

  for (int tl = 0; tl < ntiles; ++tl) {
    for (int kc = 0; kc < nch; ++kc, ++s) {
      const bool more = s + 1 < nsteps;
      const int64_t next_k0 = is_k0;
      if (more) issue();
      const unsigned char* wb = stages + (s & 1) * STAGE;
      const unsigned char* ab = wb + WBUF;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const int kb = (ks * 32 + lg * 8) * 2;
        bf16x8 wf[4];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) wf[rb] = *reinterpret_cast<const bf16x8*>(wb + (wrow(rb) + lc) * ROWB + kb);
#pragma unroll
        for (int pb = 0; pb < 4; ++pb) {
          const int px = wp * 64 + pb * 16 + lc;
          const bf16x8 ah = *reinterpret_cast<const bf16x8*>(ab + px * ROWB + kb);
#pragma unroll
          for (int rb = 0; rb < 4; ++rb) acc[pb][rb] = mfma_bf16(wf[rb], ah, acc[pb][rb]);
          if constexpr (OPM == OPM_SPLIT) {
            const bf16x8 al = *reinterpret_cast<const bf16x8*>(ab + LT_P * ROWB + px * ROWB + kb);
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) acc[pb][rb] = mfma_bf16(wf[rb], al, acc[pb][rb]);
          }
        }
      }
      if (kc + 1 < nch && more) {  // the tile continues: stage the next chunk now
        commit((s + 1) & 1, next_k0);
        advance_issue();
        __syncthreads();
      }
    }

    // ---- epilogue of the tile (the next tile's first chunk is in registers)
    {
      const int t = t0 + tl * per;
      const int pt = t / ntn, nt = t - pt * ntn;
      const int e0 = wn * WCH + lg * RUN;
      const int64_t run0 = (int64_t)nt * TNO + e0;
      const bool full_n = run0 + RUN <= p.n;
      float b1[RUN], b2[GATE ? RUN : 1], sc[RUN];
#pragma unroll
      for (int i = 0; i < RUN; ++i) {
        const bool ok = run0 + i < p.n;
        b1[i] = (p.bias && ok) ? p.bias[run0 + i] : 0.f;
        if constexpr (GATE) b2[i] = (p.bias && ok) ? p.bias[p.n + run0 + i] : 0.f;
        sc[i] = ((p.scale && ok) ? p.scale[run0 + i] : 1.f) * p.out_scale;
      }
#pragma unroll
      for (int pb = 0; pb < 4; ++pb) {
        const int64_t q = (int64_t)pt * LT_P + wp * 64 + pb * 16 + lc;
        float v[RUN];
        if constexpr (GATE) {
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              v[j * 4 + i] = (acc[pb][j][i] + b1[j * 4 + i]) * (acc[pb][2 + j][i] + b2[j * 4 + i]);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) v[j * 4 + i] = acc[pb][j][i] + b1[j * 4 + i];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[pb][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (q >= p.m) continue;
        if (p.act == ACT_GELU) {
#pragma unroll
          for (int i = 0; i < RUN; ++i) v[i] = gelu_erf(v[i]);
        } else if (p.act == ACT_LRELU) {
#pragma unroll
          for (int i = 0; i < RUN; ++i) v[i] = v[i] >= 0.f ? v[i] : v[i] * p.slope;
        }
#pragma unroll
        for (int i = 0; i < RUN; ++i) v[i] *= sc[i];
        int64_t oo, ro;
        if (p.c_mode == CM_SHUFFLE) {
          const int64_t hwi = (int64_t)p.h * p.w;
          const int64_t im = q / hwi;
          const int rr = (int)(q - im * hwi);
          const int y = rr / p.w, x = rr - (rr / p.w) * p.w;
          const int64_t cq = p.n >> 2;
          const int64_t qd = run0 / cq, cc = run0 - qd * cq;
          oo = ((im * 2 * p.h + 2 * y + (qd >> 1)) * 2 * p.w + 2 * x + (qd & 1)) * cq + cc;
          ro = oo;
        } else {
          oo = q * p.ldc + run0;
          ro = q * p.ldr + run0;
        }
        store_run<RUN>(p, v, oo, ro, run0, full_n);
      }
    }
    if (s < nsteps) {  // stage the next tile's first chunk (loaded during the last products)
      commit(s & 1, 0);
      advance_issue();
      __syncthreads();
    }
  }
}

}  // namespace clarus
