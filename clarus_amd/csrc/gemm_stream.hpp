// Streaming fused GEMM for NHWC rows when all of W^T fits in LDS (K <= 32 * KS).
//
// Same math and MFMA mapping as gemm_kernel (D[channel][pixel] = W^T . A^T, a lane holds 4 * NB
// consecutive output channels of one pixel), different schedule, built for the HBM-bound
// shapes where the A stream and the output dominate:
//   * the workgroup copies W^T rows [n0, n0 + TN) (+ the gate half), all K, into LDS once
//     (direct global->LDS copies) and never synchronises again;
//   * each wave independently walks 16-pixel blocks b = wave_id, wave_id + S, ... (S = number of
//     waves in the grid), double-buffered in registers: the next block's A (and residual) loads
//     are issued before the current block computes, and a block's stores are issued after the
//     next block's loads;
//   * prologues (LayerNorm / RMS from the row in registers, local-mean multiply, LN * m) and
//     the whole epilogue are applied per block, stores are 16-byte vectors of the lane's run.
#pragma once

#include "gemm_kernel.hpp"

namespace clarus {

// W^T row in LDS: KS * 32 elements + a 16-byte pad (bf16, or fp32 with OPM_F32)
__host__ __device__ constexpr int stream_wes(int opm) { return opm == 2 ? 4 : 2; }
__host__ __device__ constexpr int stream_wrow_elems(int ks, int opm) { return ks * 32 + 16 / stream_wes(opm); }
__host__ __device__ constexpr int stream_lds_bytes(int nb, bool gate, int ks, int opm) {
  return gemm_epi_bytes(nb) + (gate ? 2 : 1) * nb * 16 * stream_wrow_elems(ks, opm) * stream_wes(opm);
}

// register budget per lane: accumulators + D blocks of A (+ second operand) + epilogue;
// the occupancy hint keeps the compiler from hoisting beyond it
__host__ __device__ constexpr int stream_waves_per_eu(int nb, bool gate, int ks, int d, int ta, bool x2) {
  const int regs = nb * 4 * (gate ? 2 : 1) + d * ks * (ta == DT_BF16 ? 4 : 8) + (x2 ? d * ks * 8 : 0) + 72;
  return regs <= 128 ? 4 : (regs <= 168 ? 3 : 2);
}

template <int NB, bool GATE, int OPM, int TA, int KS, bool X2>
__global__ void __launch_bounds__(256)
gemm_stream_kernel(const GemmP p) {
  constexpr int G = GATE ? 2 : 1;
  constexpr int TN = NB * 16;
  constexpr int RUN = 4 * NB;
  constexpr int WES = stream_wes(OPM);
  constexpr int ROWE = stream_wrow_elems(KS, OPM);
  constexpr int ROWB = ROWE * WES;
  constexpr int WB = G * TN * ROWB;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  float* epi = reinterpret_cast<float*>(lds);
  unsigned char* wlds = lds + gemm_epi_bytes(NB);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lc = lane & 15, lg = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.y * TN;
  const int64_t bz = blockIdx.z;
  const int64_t run0 = n0 + lg * RUN;
  const int64_t K = p.k;
  const unsigned char* A = (const unsigned char*)p.a + bz * p.a_bs * esz<TA>();
  const unsigned char* Wt = (const unsigned char*)p.wt + bz * p.w_bs * WES;

  // ---- epilogue vectors and W^T rows (all of K) -> LDS, once
  for (int i = tid; i < (G + 1) * TN; i += 256) {
    const int part = i / TN;
    const int64_t c = n0 + (i - part * TN);
    float v;
    if (part < G) v = (p.bias && c < p.n) ? p.bias[part * p.n + c] : 0.f;
    else v = ((p.scale && c < p.n) ? p.scale[c] : 1.f) * p.out_scale;
    epi[i] = v;
  }
  for (int base = wave * 1024; base < WB; base += 4 * 1024) {
    const int pos = base + lane * 16;
    if (pos < WB) {
      const int r = pos / ROWB;
      int cb = pos - r * ROWB;
      if (cb >= KS * 32 * WES) cb = 0;
      const int half = r / TN;
      const int rr = r - half * TN;
      int64_t ch = n0 + ((rr & 15) >> 2) * RUN + (rr >> 4) * 4 + (rr & 3);
      if (ch > p.n - 1) ch = p.n - 1;
      int64_t kk = cb / WES;
      if (kk > K - 16 / WES) kk = K - 16 / WES;
      const unsigned char* src = Wt + ((half * p.n + ch) * K + kk) * WES;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                       (__attribute__((address_space(3))) void*)(wlds + base), 16, 0, 0);
    }
  }
  wait_vmem_all();
  __syncthreads();

  const bool lane_full = run0 + RUN <= p.n;  // this lane's whole channel run exists
  const int64_t nblk = cdiv(p.m, 16);
  const int64_t stride = (int64_t)gridDim.x * 4;
  const int64_t wid = (int64_t)blockIdx.x * 4 + wave;
  const bool stats = OPM != OPM_BF16 && (p.pro == PRO_LN || p.pro == PRO_LNMUL || p.pro == PRO_RMS);
  const float invk = 1.0f / (float)K;

  // per-pixel offset (elements) of the second prologue operand row: local-mean map / LN*m rows
  auto x2row = [&](int64_t q) __attribute__((always_inline)) -> int64_t {
    if (p.pro == PRO_MUL) {
      const int hwi = p.h * p.w;
      const int64_t im = q / hwi;
      const int rr = (int)(q - im * hwi);
      const int yq = rr / p.w;
      int sy = yq - p.pt, sx = rr - yq * p.w - p.pl;
      sy = sy < 0 ? 0 : (sy > p.oh - 1 ? p.oh - 1 : sy);
      sx = sx < 0 ? 0 : (sx > p.ow - 1 ? p.ow - 1 : sx);
      return ((im * p.oh + sy) * p.ow + sx) * K;
    }
    return q * p.ldm2;
  };

  // ---- double-buffered schedule (slots 0 / 1), per block:
  //   wait for every outstanding memory op (this slot's loads were issued a whole block ago)
  //   -> issue the next block's loads into the other slot -> issue the previous block's stores
  //   -> compute this block into packed registers.
  // The compiler sees the explicit wait, so it needs no conservative one of its own inside.
  RawFrag<TA> raw[2][KS];
  RawFrag<DT_F32> x2[X2 ? 2 : 1][X2 ? KS : 1];
  // prefetched residual of the block in each slot, raw bits: bf16 uses the first RUN / 8
  // vectors (8 values each), fp32 all RUN / 4 (4 values each)
  u32x4 rs[2][RUN / 4];
  u32x4 outv[RUN / 4];    // output of the previous block, raw bits in the same packing
  int64_t out_off = -1;   // element offset of the previous block's run (-1: none)

  auto out_offsets = [&](int64_t q, int64_t& oo, int64_t& ro) __attribute__((always_inline)) {
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
      oo = bz * p.c_bs + q * p.ldc + run0;
      ro = bz * p.r_bs + q * p.ldr + run0;
    }
  };
  const bool fast = lane_full && p.vec_out && (!p.has_res || p.vec_res);

  auto load_block = [&](int sl, int64_t blk) __attribute__((always_inline)) {
    const int64_t q = blk * 16 + lc;
    const bool ok = blk < nblk && q < p.m;
    const unsigned char* row = A + (ok ? q : 0) * p.lda * esz<TA>();
    int64_t xo = 0;
    if constexpr (X2) xo = ok ? x2row(q) : 0;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int64_t k = ks * 32 + lg * 8;
      const bool kok = ok && k < K;
      raw[sl][ks] = kok ? raw_load<TA>(row + k * esz<TA>()) : raw_zero<TA>();
      if constexpr (X2) {
        const int dt = (p.pro == PRO_MUL) ? p.s_dt : p.m2_dt;
        const unsigned char* base = (const unsigned char*)((p.pro == PRO_MUL) ? p.small : p.m2);
        RawFrag<DT_F32> v;
        v.a = v.b = f32x4{0.f, 0.f, 0.f, 0.f};
        if (kok) {
          if (dt == DT_BF16) {
            const f32x8 t = load8<DT_BF16>(base + (xo + k) * 2);
            v.a = f32x4{t.v[0], t.v[1], t.v[2], t.v[3]};
            v.b = f32x4{t.v[4], t.v[5], t.v[6], t.v[7]};
          } else {
            v.a = reinterpret_cast<const f32x4*>(base + (xo + k) * 4)[0];
            v.b = reinterpret_cast<const f32x4*>(base + (xo + k) * 4)[1];
          }
        }
        x2[sl][ks] = v;
      }
    }
    if (p.has_res && fast && ok) {
      int64_t oo, ro;
      out_offsets(q, oo, ro);
      if (p.r_dt == DT_BF16) {
        const unsigned short* rp = (const unsigned short*)p.res + ro;
#pragma unroll
        for (int j = 0; j < RUN / 8; ++j) {
          const u32x2 a = *reinterpret_cast<const u32x2*>(rp + 8 * j);
          const u32x2 b = *reinterpret_cast<const u32x2*>(rp + 8 * j + 4);
          rs[sl][j] = u32x4{a[0], a[1], b[0], b[1]};
        }
      } else {
        const float* rp = (const float*)p.res + ro;
#pragma unroll
        for (int j = 0; j < RUN / 4; ++j) rs[sl][j] = *reinterpret_cast<const u32x4*>(rp + 4 * j);
      }
    }
  };

  auto flush_out = [&]() __attribute__((always_inline)) {  // stores of the previous block (fast path only)
    if (out_off < 0) return;
    if (p.c_dt == DT_BF16) {
      unsigned short* op = (unsigned short*)p.c + out_off;
      if (RUN >= 8 && p.vec_out == 2) {
#pragma unroll
        for (int j = 0; j < RUN / 8; ++j) *reinterpret_cast<u32x4*>(op + 8 * j) = outv[j];
      } else {
#pragma unroll
        for (int j = 0; j < RUN / 8; ++j) {
          *reinterpret_cast<u32x2*>(op + 8 * j) = u32x2{outv[j][0], outv[j][1]};
          *reinterpret_cast<u32x2*>(op + 8 * j + 4) = u32x2{outv[j][2], outv[j][3]};
        }
      }
    } else {
      float* op = (float*)p.c + out_off;
#pragma unroll
      for (int j = 0; j < RUN / 4; ++j) *reinterpret_cast<u32x4*>(op + 4 * j) = outv[j];
    }
    out_off = -1;
  };

  auto compute_block = [&](int sl, int64_t blk) __attribute__((always_inline)) {
    // compiler-only barrier: re-read the W fragments from LDS for every block instead of
    // hoisting all of them into registers (which would cost occupancy)
    asm volatile("" ::: "memory");
    const int64_t q = blk * 16 + lc;
    const bool pv = q < p.m;
    float mean = 0.f, rstd = 1.f;
    if (stats) {  // row statistics from the registers (exact two-pass)
      float s = 0.f;
      if (p.pro != PRO_RMS) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const f32x8 a = raw_f32<TA>(raw[sl][ks]);
#pragma unroll
          for (int i = 0; i < 8; ++i) s += a.v[i];
        }
        mean = sum_col4(s) * invk;
      }
      float ss = 0.f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (ks * 32 + lg * 8 >= K) continue;
        const f32x8 a = raw_f32<TA>(raw[sl][ks]);
#pragma unroll
        for (int i = 0; i < 8; ++i) { const float t = a.v[i] - mean; ss += t * t; }
      }
      rstd = rsqrtf(sum_col4(ss) * invk + p.ln_eps);
    }
    f32x4 acc[NB], acc2[GATE ? NB : 1];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (GATE) acc2[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bf16x8 hi, lo;
      f32x8 a;
      if constexpr (OPM == OPM_BF16) {
        hi = __builtin_bit_cast(bf16x8, raw[sl][ks].q);
      } else {
        a = raw_f32<TA>(raw[sl][ks]);
        const int64_t k = ks * 32 + lg * 8;
        if (p.pro == PRO_LN) {
#pragma unroll
          for (int i = 0; i < 8; ++i) a.v[i] = (a.v[i] - mean) * rstd;
        } else if (p.pro == PRO_RMS) {
#pragma unroll
          for (int i = 0; i < 8; ++i) a.v[i] = a.v[i] * rstd;
        }
        if constexpr (X2) {
          const f32x8 m = raw_f32<DT_F32>(x2[sl][ks]);
          if (p.pro == PRO_MUL) {
#pragma unroll
            for (int i = 0; i < 8; ++i) a.v[i] *= m.v[i];
          } else {  // PRO_LNMUL
            const bool kok = k < K;
            const f32x8 lw = kok ? load8<DT_F32>(p.lnw + k) : zero8();
            const f32x8 lb = kok ? load8<DT_F32>(p.lnb + k) : zero8();
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const float mm = (p.m2_act == ACT_GELU) ? gelu_erf(m.v[i]) : m.v[i];
              a.v[i] = (((a.v[i] - mean) * rstd) * lw.v[i] + lb.v[i]) * mm;
            }
          }
        }
        if (!(pv && k < K)) a = zero8();
        if constexpr (OPM == OPM_SPLIT) split_bf16(a, hi, lo);
      }
#pragma unroll
      for (int j = 0; j < NB; ++j) {
#pragma unroll
        for (int hf = 0; hf < G; ++hf) {
          const unsigned char* wp = wlds + (size_t)(hf * TN + j * 16 + lc) * ROWB + (ks * 32 + lg * 8) * WES;
          f32x4 t = hf ? acc2[GATE ? j : 0] : acc[j];
          if constexpr (OPM == OPM_F32) {  // fp32 products: mfma i contracts k = ks * 32 + 8 lg + i over lg
            const f32x4 w0 = *reinterpret_cast<const f32x4*>(wp);
            const f32x4 w1 = *reinterpret_cast<const f32x4*>(wp + 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) t = mfma_f32(w0[i], a.v[i], t);
#pragma unroll
            for (int i = 0; i < 4; ++i) t = mfma_f32(w1[i], a.v[4 + i], t);
          } else {
            const bf16x8 wv = *reinterpret_cast<const bf16x8*>(wp);
            t = mfma_bf16(wv, hi, t);
            if constexpr (OPM == OPM_SPLIT) t = mfma_bf16(wv, lo, t);
          }
          if (hf) acc2[GATE ? j : 0] = t; else acc[j] = t;
        }
      }
    }
    if (!pv) return;
    // ---- epilogue math
    float v[RUN];
    const int e0 = lg * RUN;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(epi + e0 + j * 4);
      f32x4 b2 = b1;
      if constexpr (GATE) b2 = *reinterpret_cast<const f32x4*>(epi + TN + e0 + j * 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float x = acc[j][i] + b1[i];
        if constexpr (GATE) x = x * (acc2[j][i] + b2[i]);
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
    int64_t oo, ro;
    out_offsets(q, oo, ro);
    if (fast) {
      if (p.has_res) {
        if (p.r_dt == DT_BF16) {
#pragma unroll
          for (int j = 0; j < RUN / 8; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              v[8 * j + 2 * i] += __uint_as_float(rs[sl][j][i] << 16);
              v[8 * j + 2 * i + 1] += __uint_as_float(rs[sl][j][i] & 0xffff0000u);
            }
        } else {
#pragma unroll
          for (int j = 0; j < RUN / 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) v[4 * j + i] += __uint_as_float(rs[sl][j][i]);
        }
      }
      if (p.c_dt == DT_BF16) {
#pragma unroll
        for (int j = 0; j < RUN / 8; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            outv[j][i] = (unsigned)f32_to_bf16_bits(v[8 * j + 2 * i]) |
                         ((unsigned)f32_to_bf16_bits(v[8 * j + 2 * i + 1]) << 16);
      } else {
#pragma unroll
        for (int j = 0; j < RUN / 4; ++j)
          outv[j] = u32x4{__float_as_uint(v[4 * j]), __float_as_uint(v[4 * j + 1]), __float_as_uint(v[4 * j + 2]),
                          __float_as_uint(v[4 * j + 3])};
      }
      out_off = oo;  // stored after the next block's loads are issued
    } else {          // partial channel tile / unaligned output: element-wise, immediately
#pragma unroll
      for (int i = 0; i < RUN; ++i) {
        if (run0 + i >= p.n) continue;
        float x = v[i];
        if (p.has_res) x += load1(p.res, p.r_dt, ro + i);
        store1(p.c, p.c_dt, oo + i, x);
      }
    }
  };

  if (wid < nblk) load_block(0, wid);
  for (int64_t blk = wid; blk < nblk; blk += 2 * stride) {
    wait_vmem_all();
    if (blk + stride < nblk) load_block(1, blk + stride);
    flush_out();
    compute_block(0, blk);
    if (blk + stride >= nblk) break;
    wait_vmem_all();
    if (blk + 2 * stride < nblk) load_block(0, blk + 2 * stride);
    flush_out();
    compute_block(1, blk + stride);
  }
  flush_out();
}

}  // namespace clarus
