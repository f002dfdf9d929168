// Streaming fused GEMM with an LDS ring per wave (NHWC rows, short K; LN / RMS / TLC map
// prologues; row or pixel-shuffle output), gfx950.
//
// Same math, MFMA mapping and epilogue as gemm_stream_kernel (D[channel][pixel] = W^T . A^T on
// 16x16 MFMAs, a lane holds 4 * NB consecutive output channels of one pixel, all of W^T for the
// workgroup's channel tile resident in LDS). What changes is how A reaches the MFMAs:
//   * gemm_stream_kernel keeps the next 16-pixel block in registers, one block per wave in
//     flight. With 160-250 VGPRs it runs 2-3 waves per SIMD, so a CU holds 16-24 KiB of A in
//     flight: at HBM latency that caps the stream near 4 TB/s (measured: c64 expand 4.3 TB/s,
//     c128 expand 2.9 TB/s);
//   * here every wave owns a ring of RS_DEPTH (2-4, what fits in LDS next to W^T) blocks,
//     filled by direct global -> LDS copies (16 bytes per lane), so RS_DEPTH - 1 blocks are in
//     flight without costing registers. The residual block travels in the same ring. Waits are
//     per-wave vmcnt counts (the copies complete in issue order; stores only add to the count):
//     at block b the copies of blocks b + 1 .. b + RS_DEPTH - 2 may stay in flight. No
//     workgroup barrier after W is staged.
// Ring slot of a block: 16 pixel rows of RB bytes (A, K padded to 32 * KS elements) followed by
// 16 rows of residual. Row r stores its 16-byte unit u at slot u ^ f(r), f(r) = (r / (256 /
// RB)) % U (U units per row): the 16 lanes reading one unit of 16 consecutive rows hit 16
// distinct 16-byte bank groups. Units past K (and rows past M) are copied from clamped
// addresses and masked when read.
#pragma once

#include "gemm_stream.hpp"

namespace clarus {

constexpr int RS_MAX_DEPTH = 4;  // ring blocks per wave, at most

// pixels per ring block (16 or 32; with 32 two 16-pixel MFMA halves share each W^T fragment
// read, which halves W^T LDS traffic but doubles the slot: measured slower on every NAFNet,
// config-1 and attn . V shape but the widest, e.g. attn . V fp32 l0 137 vs 124 us)
constexpr int RS_BP = 16;

template <int KS, int TA>
struct RsA {
  static constexpr int ES = TA == DT_BF16 ? 2 : 4;
  static constexpr int RB = KS * 32 * ES;       // bytes per A row in the ring
  static constexpr int U = RB / 16;             // 16-byte units per row
  static constexpr int RPB = RB >= 256 ? 1 : 256 / RB;  // rows per 256-byte bank row
  static constexpr int BYTES = RS_BP * RB;      // one block of A
};

// residual bytes per block row: the workgroup's TN channels
template <int NB, int RDT>
struct RsR {
  static constexpr int ES = RDT == DT_BF16 ? 2 : 4;
  static constexpr int RB = NB * 16 * ES;
  static constexpr int U = RB / 16;
  static constexpr int RPB = RB >= 256 ? 1 : 256 / RB;
  static constexpr int BYTES = RS_BP * RB;
};

template <int U, int RPB>
__device__ __forceinline__ int rs_slot(int row, int unit) { return unit ^ ((row / RPB) & (U - 1)); }

// one ring slot: A rows, the prologue's map rows (bf16, X2), the residual rows
__host__ __device__ constexpr int rowstream_slot_bytes(int nb, int ks, int ta, int rdt, bool res, bool x2 = false) {
  return RS_BP * (ks * 32 * (ta == DT_BF16 ? 2 : 4) + (x2 ? ks * 32 * 2 : 0) + (res ? nb * 16 * (rdt == DT_BF16 ? 2 : 4) : 0));
}
// Shape of the workgroup: NW waves sharing one copy of W^T, each with a ring of depth D, chosen
// for the most blocks in flight per CU:
//   * 4 waves with a ring of at least 3 while two workgroups still share a CU (80 KiB each);
//   * else 8 waves with a ring of at least 3 in one workgroup per CU (160 KiB): a large W^T
//     tile (K = 128 with a gate: 35 KiB) is then staged once for 8 waves instead of twice;
//   * else 4 waves with a ring of 2 in two workgroups per CU, or one workgroup with what fits.
// One workgroup of 4 waves with a deeper ring measured slower than two with a ring of 2
// (c128 expand 51.8 vs 38.6 us). Below a depth of 2 the shape has no kernel.
struct RsShape {
  int nw, depth;
};
__host__ __device__ constexpr RsShape rowstream_shape(int nb, bool gate, int ks, int opm, int ta, int rdt, bool res,
                                                      bool x2 = false) {
  const int slot = rowstream_slot_bytes(nb, ks, ta, rdt, res, x2);
  const int w = stream_lds_bytes(nb, gate, ks, opm);
  auto cap = [](int d) { return d > RS_MAX_DEPTH ? RS_MAX_DEPTH : d; };
  const int d4 = cap((80 * 1024 - w) / (4 * slot));
  if (d4 >= 3) return RsShape{4, d4};
  const int d8 = cap((160 * 1024 - w) / (8 * slot));
  if (d8 >= 3) return RsShape{8, d8};
  if (d4 >= 2) return RsShape{4, d4};
  return RsShape{4, cap((160 * 1024 - w) / (4 * slot))};
}
__host__ __device__ constexpr int rowstream_depth(int nb, bool gate, int ks, int opm, int ta, int rdt, bool res,
                                                  bool x2 = false) {
  return rowstream_shape(nb, gate, ks, opm, ta, rdt, res, x2).depth;
}
__host__ __device__ constexpr int rowstream_waves(int nb, bool gate, int ks, int opm, int ta, int rdt, bool res,
                                                  bool x2 = false) {
  return rowstream_shape(nb, gate, ks, opm, ta, rdt, res, x2).nw;
}
__host__ __device__ constexpr int rowstream_lds_bytes(int nb, bool gate, int ks, int opm, int ta, int rdt, bool res,
                                                      bool x2 = false) {
  const RsShape sh = rowstream_shape(nb, gate, ks, opm, ta, rdt, res, x2);
  return stream_lds_bytes(nb, gate, ks, opm) + sh.nw * sh.depth * rowstream_slot_bytes(nb, ks, ta, rdt, res, x2);
}

// RDT: residual dtype (ignored when RES is false). X2: the TLC map multiply prologue (bf16 map
// rows gathered into the ring); LN / RMS prologues (runtime p.pro) take their statistics from
// the row in registers. Prologues come with OPM_SPLIT (the fp32 prologue output as hi + lo).
template <int NB, bool GATE, int OPM, int TA, int KS, bool RES, int RDT, bool X2 = false>
__global__ void __launch_bounds__(64 * rowstream_waves(NB, GATE, KS, OPM, TA, RDT, RES, X2))
gemm_rowstream_kernel(const GemmP p) {
  constexpr int NW = rowstream_waves(NB, GATE, KS, OPM, TA, RDT, RES, X2);  // waves per workgroup
  constexpr int NT = 64 * NW;
  constexpr int BP = RS_BP;
  constexpr int HB = BP / 16;  // 16-pixel MFMA halves per ring block
  constexpr int G = GATE ? 2 : 1;
  constexpr int TN = NB * 16;
  constexpr int RUN = 4 * NB;
  constexpr int WES = stream_wes(OPM);
  constexpr int ROWE = stream_wrow_elems(KS, OPM);
  constexpr int ROWB = ROWE * WES;
  constexpr int WB = G * TN * ROWB;
  using AL = RsA<KS, TA>;
  using RL = RsR<NB, RDT>;
  using ML = RsA<KS, DT_BF16>;                  // map rows (X2): same units as bf16 A rows
  constexpr int MOFF = AL::BYTES;               // map block offset in a slot
  constexpr int ROFF = AL::BYTES + (X2 ? ML::BYTES : 0);  // residual block offset
  constexpr int SLOT = ROFF + (RES ? RL::BYTES : 0);
  constexpr int CA = AL::BYTES / 1024;          // A copies per lane per block
  constexpr int CM = X2 ? ML::BYTES / 1024 : 0;  // map copies per lane per block
  constexpr int CR = RES ? RL::BYTES / 1024 : 0;  // residual copies per lane per block
  static_assert(AL::BYTES % 1024 == 0 && (!RES || RL::BYTES % 1024 == 0) && (!X2 || ML::BYTES % 1024 == 0),
                "blocks are whole copy instructions");
  static_assert(!X2 || OPM == OPM_SPLIT || OPM == OPM_ROUND, "a prologue output is split or rounded to bf16");
  constexpr int C = CA + CM + CR;               // copy instructions per block
  constexpr int RS_DEPTH = rowstream_depth(NB, GATE, KS, OPM, TA, RDT, RES, X2);
  static_assert(RS_DEPTH >= 2 && RS_DEPTH <= 4, "ring depth");
  static_assert(2 * C < 64, "vmcnt range");
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  float* epi = reinterpret_cast<float*>(lds);
  unsigned char* wlds = lds + gemm_epi_bytes(NB);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lc = lane & 15, lg = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.y * TN;
  const int64_t bz = blockIdx.z;
  const int64_t run0 = n0 + lg * RUN;
  const int64_t K = p.k;
  const unsigned char* A = (const unsigned char*)p.a + bz * p.a_bs * AL::ES;
  const unsigned char* Wt = (const unsigned char*)p.wt + bz * p.w_bs * WES;
  unsigned char* ring = wlds + WB + wave * (RS_DEPTH * SLOT);

  // ---- epilogue vectors and W^T rows (all of K) -> LDS, once (as gemm_stream_kernel)
  for (int i = tid; i < (G + 1) * TN; i += NT) {
    const int part = i / TN;
    const int64_t c = n0 + (i - part * TN);
    float v;
    if (part < G) v = (p.bias && c < p.n) ? p.bias[part * p.n + c] : 0.f;
    else v = ((p.scale && c < p.n) ? p.scale[c] : 1.f) * p.out_scale;
    epi[i] = v;
  }
  for (int base = wave * 1024; base < WB; base += NW * 1024) {
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

  const bool lane_full = run0 + RUN <= p.n;
  const int64_t nblk = cdiv(p.m, BP);
  const int64_t stride = (int64_t)gridDim.x * NW;
  const int64_t wid = (int64_t)blockIdx.x * NW + wave;
  const int64_t nmine = wid < nblk ? (nblk - 1 - wid) / stride + 1 : 0;  // blocks of this wave
  const int ua_valid = (int)(K * AL::ES / 16);  // A units per row that hold k < K
  const int ua_map = (int)(K * 2 / 16);         // map units per row that hold k < K

  // element offset of (pixel q, channel c of the N space) in the output, which the residual
  // shares under the pixel shuffle (N = (dy, dx, c'), output [*, 2h, 2w, N / 4])
  auto shuffled = [&](int64_t q, int64_t c) __attribute__((always_inline)) -> int64_t {
    const int64_t hwi = (int64_t)p.h * p.w;
    const int64_t im = q / hwi;
    const int rr = (int)(q - im * hwi);
    const int y = rr / p.w, x = rr - (rr / p.w) * p.w;
    const int64_t cq = p.n >> 2;
    const int64_t qd = c / cq, cc = c - qd * cq;
    return ((im * 2 * p.h + 2 * y + (qd >> 1)) * 2 * p.w + 2 * x + (qd & 1)) * cq + cc;
  };
  auto out_offsets = [&](int64_t q, int64_t& oo, int64_t& ro) __attribute__((always_inline)) {
    if (p.c_mode == CM_SHUFFLE) {
      oo = shuffled(q, run0);
      ro = oo;
    } else {
      oo = bz * p.c_bs + q * p.ldc + run0;
      ro = bz * p.r_bs + q * p.ldr + run0;
    }
  };
  const bool fast = lane_full && p.vec_out && (!RES || p.vec_res);

  // copies of block j (the wave's j-th block) into ring slot j % RS_DEPTH: copy instruction c
  // covers 64 / U rows of the block, lane i row (64 c + i) / U, slot (64 c + i) % U
  auto issue = [&](int64_t j) __attribute__((always_inline)) {
    const int64_t blk = wid + j * stride;
    unsigned char* slot = ring + (int)(j % RS_DEPTH) * SLOT;
#pragma unroll
    for (int c = 0; c < CA; ++c) {
      const int idx = c * 64 + lane;
      const int row = idx / AL::U, s = idx - row * AL::U;
      int u = rs_slot<AL::U, AL::RPB>(row, s);
      if (u > ua_valid - 1) u = ua_valid - 1;  // past K: any valid unit (masked when read)
      int64_t q = blk * BP + row;
      if (q > p.m - 1) q = p.m - 1;            // past M: any valid row (not stored)
      const unsigned char* src = A + (q * p.lda) * AL::ES + u * 16;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                       (__attribute__((address_space(3))) void*)(slot + c * 1024), 16, 0, 0);
    }
    if constexpr (X2) {  // map row of each pixel: S[clamp(y - pt), clamp(x - pl)], all K channels
      unsigned char* mslot = slot + MOFF;
#pragma unroll
      for (int c = 0; c < CM; ++c) {
        const int idx = c * 64 + lane;
        const int row = idx / ML::U, s = idx - row * ML::U;
        int u = rs_slot<ML::U, ML::RPB>(row, s);
        if (u > ua_map - 1) u = ua_map - 1;
        int64_t q = blk * BP + row;
        if (q > p.m - 1) q = p.m - 1;
        const int hwi = p.h * p.w;
        const int64_t im = q / hwi;
        const int rr = (int)(q - im * hwi);
        const int yq = rr / p.w;
        int sy = yq - p.pt, sx = rr - yq * p.w - p.pl;
        sy = sy < 0 ? 0 : (sy > p.oh - 1 ? p.oh - 1 : sy);
        sx = sx < 0 ? 0 : (sx > p.ow - 1 ? p.ow - 1 : sx);
        const unsigned char* src = (const unsigned char*)p.small + (((im * p.oh + sy) * p.ow + sx) * K) * 2 + u * 16;
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                         (__attribute__((address_space(3))) void*)(mslot + c * 1024), 16, 0, 0);
      }
    }
    if constexpr (RES) {
      unsigned char* rslot = slot + ROFF;
#pragma unroll
      for (int c = 0; c < CR; ++c) {
        const int idx = c * 64 + lane;
        const int row = idx / RL::U, s = idx - row * RL::U;
        const int u = rs_slot<RL::U, RL::RPB>(row, s);
        int64_t q = blk * BP + row;
        if (q > p.m - 1) q = p.m - 1;
        int64_t ch = n0 + u * (16 / RL::ES);
        if (ch > p.n - 16 / RL::ES) ch = p.n - 16 / RL::ES;  // channels past N: not stored
        const int64_t ro = p.c_mode == CM_SHUFFLE ? shuffled(q, ch) : bz * p.r_bs + q * p.ldr + ch;
        const unsigned char* src = (const unsigned char*)p.res + ro * RL::ES;
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                         (__attribute__((address_space(3))) void*)(rslot + c * 1024), 16, 0, 0);
      }
    }
  };

  auto compute_block = [&](int64_t j) __attribute__((always_inline)) {
    const int64_t blk = wid + j * stride;
    const unsigned char* slot = ring + (int)(j % RS_DEPTH) * SLOT;
    f32x4 acc[HB][NB], acc2[HB][GATE ? NB : 1];
#pragma unroll
    for (int h = 0; h < HB; ++h)
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        acc[h][i] = f32x4{0.f, 0.f, 0.f, 0.f};
        if constexpr (GATE) acc2[h][i] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    // this lane's 8 consecutive k of pixel 16 h + lc per k-step, from the ring (k >= K read as 0)
    RawFrag<TA> raw[HB][KS];
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      const int row = 16 * h + lc;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int64_t k = ks * 32 + lg * 8;
        const bool kok = k < K;
        if constexpr (TA == DT_BF16) {
          const int u = (int)(k / 8);
          raw[h][ks].q = kok ? *reinterpret_cast<const u32x4*>(slot + row * AL::RB + rs_slot<AL::U, AL::RPB>(row, u) * 16)
                             : u32x4{0u, 0u, 0u, 0u};
        } else {
          const int u = (int)(k / 4);
          raw[h][ks].a = kok ? *reinterpret_cast<const f32x4*>(slot + row * AL::RB + rs_slot<AL::U, AL::RPB>(row, u) * 16)
                             : f32x4{0.f, 0.f, 0.f, 0.f};
          raw[h][ks].b = kok ? *reinterpret_cast<const f32x4*>(slot + row * AL::RB +
                                                                 rs_slot<AL::U, AL::RPB>(row, u + 1) * 16)
                             : f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
    // LN / RMS statistics over each row: this lane's fragments, then the 4 lanes of the pixel
    // (exact two-pass, fixed order)
    float mean[HB], rstd[HB];
    const bool stats = (OPM == OPM_SPLIT || OPM == OPM_ROUND) && (p.pro == PRO_LN || p.pro == PRO_RMS);
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      mean[h] = 0.f;
      rstd[h] = 1.f;
      if (!stats) continue;
      const float invk = 1.0f / (float)K;
      if (p.pro == PRO_LN) {
        float sum = 0.f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const f32x8 t = raw_f32<TA>(raw[h][ks]);
#pragma unroll
          for (int i = 0; i < 8; ++i) sum += t.v[i];
        }
        mean[h] = sum_col4(sum) * invk;
      }
      float ss = 0.f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (ks * 32 + lg * 8 >= K) continue;
        const f32x8 t = raw_f32<TA>(raw[h][ks]);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float d = t.v[i] - mean[h];
          ss += d * d;
        }
      }
      rstd[h] = rsqrtf(sum_col4(ss) * invk + p.ln_eps);
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int64_t k = ks * 32 + lg * 8;
      const bool kok = k < K;
      bf16x8 hi[HB], lo[HB];
      f32x8 a[HB];
#pragma unroll
      for (int h = 0; h < HB; ++h) {
        if constexpr (OPM == OPM_BF16) {
          hi[h] = __builtin_bit_cast(bf16x8, raw[h][ks].q);
        } else {
          a[h] = raw_f32<TA>(raw[h][ks]);
          if (stats) {
#pragma unroll
            for (int i = 0; i < 8; ++i) a[h].v[i] = (a[h].v[i] - mean[h]) * rstd[h];
          }
          if constexpr (X2) {
            const int row = 16 * h + lc;
            const u32x4 mq = kok ? *reinterpret_cast<const u32x4*>(slot + MOFF + row * ML::RB +
                                                                    rs_slot<ML::U, ML::RPB>(row, (int)(k / 8)) * 16)
                                 : u32x4{0u, 0u, 0u, 0u};
            RawFrag<DT_BF16> mr;
            mr.q = mq;
            const f32x8 mv = raw_f32<DT_BF16>(mr);
#pragma unroll
            for (int i = 0; i < 8; ++i) a[h].v[i] *= mv.v[i];
          }
          if (!kok) a[h] = zero8();
          if constexpr (OPM == OPM_SPLIT) split_bf16(a[h], hi[h], lo[h]);
          if constexpr (OPM == OPM_ROUND) hi[h] = pack_bf16(a[h]);  // RNE, as the long-K prologue pass
        }
      }
      // each W^T fragment is read from LDS once for all HB pixel halves
#pragma unroll
      for (int jb = 0; jb < NB; ++jb) {
#pragma unroll
        for (int hf = 0; hf < G; ++hf) {
          const unsigned char* wp = wlds + (size_t)(hf * TN + jb * 16 + lc) * ROWB + (ks * 32 + lg * 8) * WES;
          if constexpr (OPM == OPM_F32) {  // fp32 products: mfma i contracts k = ks * 32 + 8 lg + i over lg
            const f32x4 w0 = *reinterpret_cast<const f32x4*>(wp);
            const f32x4 w1 = *reinterpret_cast<const f32x4*>(wp + 16);
#pragma unroll
            for (int h = 0; h < HB; ++h) {
              f32x4 t = hf ? acc2[h][GATE ? jb : 0] : acc[h][jb];
#pragma unroll
              for (int i = 0; i < 4; ++i) t = mfma_f32(w0[i], a[h].v[i], t);
#pragma unroll
              for (int i = 0; i < 4; ++i) t = mfma_f32(w1[i], a[h].v[4 + i], t);
              if (hf) acc2[h][GATE ? jb : 0] = t; else acc[h][jb] = t;
            }
          } else {
            const bf16x8 wv = *reinterpret_cast<const bf16x8*>(wp);
#pragma unroll
            for (int h = 0; h < HB; ++h) {
              f32x4 t = hf ? acc2[h][GATE ? jb : 0] : acc[h][jb];
              t = mfma_bf16(wv, hi[h], t);
              if constexpr (OPM == OPM_SPLIT) t = mfma_bf16(wv, lo[h], t);
              if (hf) acc2[h][GATE ? jb : 0] = t; else acc[h][jb] = t;
            }
          }
        }
      }
    }
    // ---- epilogue per pixel half
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      const int row = 16 * h + lc;
      const int64_t q = blk * BP + row;
      if (q >= p.m) continue;
      float v[RUN];
      const int e0 = lg * RUN;
#pragma unroll
      for (int jb = 0; jb < NB; ++jb) {
        const f32x4 b1 = *reinterpret_cast<const f32x4*>(epi + e0 + jb * 4);
        f32x4 b2 = b1;
        if constexpr (GATE) b2 = *reinterpret_cast<const f32x4*>(epi + TN + e0 + jb * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float x = acc[h][jb][i] + b1[i];
          if constexpr (GATE) x = x * (acc2[h][jb][i] + b2[i]);
          v[jb * 4 + i] = x;
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
      for (int jb = 0; jb < NB; ++jb) {
        const f32x4 sc = *reinterpret_cast<const f32x4*>(epi + G * TN + e0 + jb * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[jb * 4 + i] *= sc[i];
      }
      int64_t oo, ro;
      out_offsets(q, oo, ro);
      if (fast) {
        if constexpr (RES) {  // the lane's RUN residual channels from the ring
          const unsigned char* rrow = slot + ROFF + row * RL::RB;
          constexpr int PER = 16 / RL::ES;  // channels per unit
#pragma unroll
          for (int u0 = 0; u0 < RUN / PER; ++u0) {
            const int u = (lg * RUN) / PER + u0;
            const u32x4 r = *reinterpret_cast<const u32x4*>(rrow + rs_slot<RL::U, RL::RPB>(row, u) * 16);
            if constexpr (RDT == DT_BF16) {
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                v[u0 * 8 + 2 * i] += __uint_as_float(r[i] << 16);
                v[u0 * 8 + 2 * i + 1] += __uint_as_float(r[i] & 0xffff0000u);
              }
            } else {
#pragma unroll
              for (int i = 0; i < 4; ++i) v[u0 * 4 + i] += __uint_as_float(r[i]);
            }
          }
        }
        if (p.c_dt == DT_BF16) {
          unsigned short* op = (unsigned short*)p.c + oo;
#pragma unroll
          for (int jj = 0; jj < RUN / 8; ++jj) {
            u32x4 o;
#pragma unroll
            for (int i = 0; i < 4; ++i)
              o[i] = (unsigned)f32_to_bf16_bits(v[8 * jj + 2 * i]) |
                     ((unsigned)f32_to_bf16_bits(v[8 * jj + 2 * i + 1]) << 16);
            if (p.vec_out == 2) {
              *reinterpret_cast<u32x4*>(op + 8 * jj) = o;
            } else {
              *reinterpret_cast<u32x2*>(op + 8 * jj) = u32x2{o[0], o[1]};
              *reinterpret_cast<u32x2*>(op + 8 * jj + 4) = u32x2{o[2], o[3]};
            }
          }
        } else {
          float* op = (float*)p.c + oo;
#pragma unroll
          for (int jj = 0; jj < RUN / 4; ++jj)
            *reinterpret_cast<f32x4*>(op + 4 * jj) = f32x4{v[4 * jj], v[4 * jj + 1], v[4 * jj + 2], v[4 * jj + 3]};
        }
      } else {  // partial channel tile / unaligned output: element-wise
#pragma unroll
        for (int i = 0; i < RUN; ++i) {
          if (run0 + i >= p.n) continue;
          float x = v[i];
          if constexpr (RES) x += load1(p.res, p.r_dt, ro + i);
          store1(p.c, p.c_dt, oo + i, x);
        }
      }
    }
  };

  // ---- the ring: blocks 0 .. RS_DEPTH - 2 in flight before the first one is computed
  int64_t issued = 0;
  for (; issued < RS_DEPTH - 1 && issued < nmine; ++issued) issue(issued);
  for (int64_t j = 0; j < nmine; ++j) {
    // block j landed: the copies of the blocks issued after it may stay in flight (stores of
    // earlier blocks complete before them in issue order, so they are covered as well)
    const int64_t newer = issued - 1 - j;  // copy groups issued after block j's
    if (newer >= 2) wait_vmcnt<2 * C>();
    else if (newer == 1) wait_vmcnt<C>();
    else wait_vmem_all();
    // the wave's LDS reads of block j's slot come after the wait (the ring is per wave)
    asm volatile("" ::: "memory");
    if (issued < nmine) { issue(issued); ++issued; }
    compute_block(j);
  }
}

}  // namespace clarus
