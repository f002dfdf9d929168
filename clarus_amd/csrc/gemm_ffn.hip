// Fused pointwise feed-forward: clarus_hip_ffn (gfx950).
//
//   u   = SG(W1^T . pro(x) + b1)                 (2c hidden channels -> c by SimpleGate)
//   out = x + (W2^T . u + b2) * scale * out_scale
//
// for dense NHWC rows x [m][c], c = 32, 64 or 128 (bf16), with pro the row LayerNorm (no affine), the RMS
// norm or nothing. This is NAFNet's feed-forward half-block (conv4 -> SimpleGate -> conv5, the
// conv5 output scaled by gamma and added to the block input) and the fp32 pointwise chain of the
// benchmark (32 -> 64 + SimpleGate -> 32, beta * . + x).
// Unfused, the two `linear` calls move u through HBM: at NAFNet level 0 (c = 64, 720 x 1280)
// that is 118 MB written and read again, plus x read twice; here x is read once and out
// written once.
//
// Arithmetic follows the two linear calls it replaces: the normalised row is rounded once to
// bf16 for bf16 weights (the row-streaming kernel's rounding prologue), u is rounded to the
// activation dtype (bf16 activations) as the first call stores it, products accumulate in fp32
// (fp32 operands: fp32 MFMAs), and the epilogue is (acc + b2) * (scale * out_scale) + x.
//
// Mapping (32x32 MFMAs, D[row][pixel] = W^T . X^T; lane l holds D[8 (j / 4) + 4 (l / 32) + j % 4]
// [l % 32] in accumulator element j):
//   * a unit is 32 pixels; the B operand of the first product is x itself: lane l supplies pixel
//     l % 32 and, for 16-k step s, channels 16 s + 8 (l / 32) .. + 7;
//   * hidden tile T of the first product (W1^T rows 32 T .. 32 T + 31; gate partners T and
//     T + c / 32) lands in the lane as 16 values; after the gate they ARE the B operand of the
//     second product: slot i of the second product's k-step (T, a) is accumulator element 8 a + i,
//     i.e. hidden channel 32 T + 16 a + 8 (i / 4) + 4 (l / 32) + i % 4, so W2 is packed with its
//     k order permuted to match and u never leaves the registers;
//   * W2^T rows are permuted so that output element j of lane l in tile T2 is channel
//     32 T2 + 16 (j / 8) + 8 (l / 32) + j % 8: exactly the channels the lane holds of x for k-steps
//     2 T2 and 2 T2 + 1. The residual is the x fragment already in registers, and each lane
//     stores two 8-channel runs per output tile.
// Both weights are passed pre-packed in that fragment order (the host packs once per weight):
//   w1p[T][s][l][i] = w1[16 s + 8 (l / 32) + i][32 T + l % 32]          T < 2c/32, s < c/16, i < 8
//   w2p[T2][T][l][j] = w2[32 T + 8 (j / 4) + 4 (l / 32) + j % 4][o(T2, l % 32)]   j < 16
//   o(T2, r) = 32 T2 + 16 (r / 16) + 8 ((r / 4) % 2) + 4 ((r / 8) % 2) + r % 4
// with w1 [c][2c] and w2 [c][c] in the `linear` layout (input channel first).
// Data movement: one workgroup per CU (persistent) holds both packed weights and the bias / scale
// tables in LDS; each wave owns a ring of 32-pixel units of x, filled by direct global ->
// LDS copies (16 bytes per lane, whole rows per instruction, through a buffer bounded to the
// unit's rows: rows past M read as zeros), with 16-byte units of a row XOR-swizzled so that the
// fragment reads of 16 consecutive rows hit distinct bank groups. The bias vectors are the start
// values of the accumulators, and the normalised rows are computed once per unit. Output
// stores are buffer stores bounded to the unit's valid rows, so every wave issues the same
// number of memory operations per unit and the ring waits are exact vmcnt counts.
// No counterpart in the reference: it composes two `linear` calls (ops/torch_ref.py:103-130;
// models/nafnet/__init__.py:159-161 for the block; the chain of the pointwise benchmark config).
#include "capi.hpp"
#include "gemm_mfma32.hpp"

namespace clarus {

namespace {

constexpr int FF_P = 32;  // pixels per unit

__host__ __device__ constexpr int ff_es(int dt) { return dt == DT_BF16 ? 2 : 4; }
__host__ __device__ constexpr int ff_unit_bytes(int c, int dt) { return FF_P * c * ff_es(dt); }
__host__ __device__ constexpr int ff_fixed_bytes(int c, int dt) {
  return 3 * c * c * ff_es(dt) + 4 * c * 4;  // W1 [2c][c] + W2 [c][c] + b1 [2c] | b2 [c] | scale [c]
}
// 8 waves with a ring of 3 units (two in flight while one is computed) where it fits, else 4
// waves with what fits (at most 3). Measured at NAFNet level 0 (c = 64, 720 x 1280, bf16), us, x
// read from HBM / from the last-level cache (back-to-back calls): 8 waves, ring 3: 56.7 / 49.8;
// ring 4: 58.2 / 51.6; 10 waves, ring 3: 66.3 / 51.7; 12 waves, ring 2: 64.3 / 45.4; 4 waves:
// 80 / 89. The fp32 config-1 chain (c = 32): 11.6 / 10.5 with 8 waves, 13.3 / 11.9 with 12.
// c = 128 (bf16): the weights and tables take 98 KiB, which leaves one 8 KiB slot for each of 7
// waves; a wave copies its fragments of the slot's unit into registers and refills the slot with
// the next unit at once, so one unit is in flight while one is computed.
__host__ __device__ constexpr int ff_waves(int c, int dt) {
  return c == 128 ? 7 : (160 * 1024 - ff_fixed_bytes(c, dt)) / (8 * ff_unit_bytes(c, dt)) >= 3 ? 8 : 4;
}
__host__ __device__ constexpr int ff_depth(int c, int dt) {
  const int d = (160 * 1024 - ff_fixed_bytes(c, dt)) / (ff_waves(c, dt) * ff_unit_bytes(c, dt));
  return c == 128 ? 1 : d > 3 ? 3 : d;
}
__host__ __device__ constexpr int ff_lds_bytes(int c, int dt) {
  return ff_fixed_bytes(c, dt) + ff_waves(c, dt) * ff_depth(c, dt) * ff_unit_bytes(c, dt);
}
static_assert(ff_depth(64, DT_F32) >= 2 && ff_depth(64, DT_BF16) >= 2 && ff_depth(32, DT_F32) >= 2 &&
                  ff_depth(32, DT_BF16) >= 2 && ff_lds_bytes(128, DT_BF16) <= 160 * 1024,
              "LDS");

struct FfP {
  const void* x;      // [m][c]
  const void* w1p;    // packed, see above
  const void* w2p;
  const float* b1;    // [2c] or null
  const float* b2;    // [c] or null
  const float* scale; // [c] or null
  void* out;          // [m][c]
  int64_t m;
  float ln_eps, out_scale;
};

__device__ __forceinline__ f32x16 mfma32_f32(float a, float b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int ff_swz(int row, int unit, int u, int rpb) { return unit ^ ((row / rpb) & (u - 1)); }

// One 32-pixel unit from its x fragments (xr[s]: channels 16 s + 8 (lane / 32) .. + 7 of pixel
// q0 + lane % 32): the prologue, both products with the gate between them, the epilogue and
// NS buffer stores (rows past M dropped by the range).
// a lane's raw x fragment (8 consecutive channels): packed bf16, or fp32
template <int DT> struct XFragT;
template <> struct XFragT<DT_BF16> { using T = u32x4; };
template <> struct XFragT<DT_F32> { using T = f32x8; };
template <int DT>
__device__ __forceinline__ float xel(const typename XFragT<DT>::T& f, int i) {
  if constexpr (DT == DT_BF16) return __uint_as_float((i & 1) ? (f[i >> 1] & 0xffff0000u) : (f[i >> 1] << 16));
  else return f.v[i];
}

template <int C, int DT, int PRO>
__device__ __forceinline__ void ffn_unit(const typename XFragT<DT>::T (&xr)[C / 16], const unsigned char* w1l,
                                         const unsigned char* w2l, const float* tab, const FfP& p, int64_t q0,
                                         int lane) {
  constexpr int ES = ff_es(DT), RB = C * ES, KS = C / 16, TG = C / 32;
  const int px = lane & 31, hf = lane >> 5;
  // the first product's B operand: the row, LayerNorm'd ((x - mean) * rstd, two-pass) or RMS
  // normalised over the pixel's c channels (two lanes hold half each), rounded to bf16 for bf16
  // weights; the raw fragments themselves without a prologue
  f32x8 xa[KS];
  bf16x8 xb[KS];
  if constexpr (PRO == PRO_NONE) {
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if constexpr (DT == DT_BF16) xb[s] = __builtin_bit_cast(bf16x8, xr[s]);
      else xa[s] = xr[s];
    }
  } else {
    const float invc = 1.0f / (float)C;
    float mean = 0.f;
    if constexpr (PRO == PRO_LN) {
      float sum = 0.f;
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int i = 0; i < 8; ++i) sum += xel<DT>(xr[s], i);
      sum += __shfl_xor(sum, 32, 64);
      mean = sum * invc;
    }
    float ss = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        xa[s].v[i] = PRO == PRO_LN ? xel<DT>(xr[s], i) - mean : xel<DT>(xr[s], i);
        ss += xa[s].v[i] * xa[s].v[i];
      }
    ss += __shfl_xor(ss, 32, 64);
    const float rstd = rsqrtf(ss * invc + p.ln_eps);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int i = 0; i < 8; ++i) xa[s].v[i] *= rstd;
      if constexpr (DT == DT_BF16) xb[s] = pack_bf16(xa[s]);  // RNE
    }
  }

  // ---- first product, its bias in the accumulators' start values, and the gate: uf[T] holds
  // the lane's 16 gated values of hidden tile T (element 4 q + jj: hidden channel
  // 32 T + 8 q + 4 hf + jj, its gate partner c channels on)
  using UFrag = typename std::conditional<DT == DT_BF16, u32x4, f32x4>::type;
  UFrag uf[TG][DT == DT_BF16 ? 2 : 4];
#pragma unroll
  for (int T = 0; T < TG; ++T) {
    f32x16 ga, gb;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4 ba = *reinterpret_cast<const f32x4*>(tab + 32 * T + 8 * q + 4 * hf);
      const f32x4 bb = *reinterpret_cast<const f32x4*>(tab + C + 32 * T + 8 * q + 4 * hf);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        ga[4 * q + jj] = ba[jj];
        gb[4 * q + jj] = bb[jj];
      }
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if constexpr (DT == DT_BF16) {
        const bf16x8 wa = *reinterpret_cast<const bf16x8*>(w1l + ((T * KS + s) * 64 + lane) * 16);
        const bf16x8 wb = *reinterpret_cast<const bf16x8*>(w1l + (((T + TG) * KS + s) * 64 + lane) * 16);
        ga = mfma32_bf16(wa, xb[s], ga);
        gb = mfma32_bf16(wb, xb[s], gb);
      } else {
        const unsigned char* pa = w1l + ((T * KS + s) * 64 + lane) * 32;
        const unsigned char* pb = w1l + (((T + TG) * KS + s) * 64 + lane) * 32;
        const f32x4 wa0 = *reinterpret_cast<const f32x4*>(pa), wa1 = *reinterpret_cast<const f32x4*>(pa + 16);
        const f32x4 wb0 = *reinterpret_cast<const f32x4*>(pb), wb1 = *reinterpret_cast<const f32x4*>(pb + 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ga = mfma32_f32(wa0[i], xa[s].v[i], ga);
          gb = mfma32_f32(wb0[i], xa[s].v[i], gb);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ga = mfma32_f32(wa1[i], xa[s].v[4 + i], ga);
          gb = mfma32_f32(wb1[i], xa[s].v[4 + i], gb);
        }
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float g[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) g[jj] = ga[4 * q + jj] * gb[4 * q + jj];
      if constexpr (DT == DT_BF16) {
        uf[T][q / 2][2 * (q & 1)] = (unsigned)f32_to_bf16_bits(g[0]) | ((unsigned)f32_to_bf16_bits(g[1]) << 16);
        uf[T][q / 2][2 * (q & 1) + 1] = (unsigned)f32_to_bf16_bits(g[2]) | ((unsigned)f32_to_bf16_bits(g[3]) << 16);
      } else {
        uf[T][q] = f32x4{g[0], g[1], g[2], g[3]};
      }
    }
    // c = 128: keep the scheduler from hoisting the next tiles' weight fragments (spills)
    if constexpr (C >= 128) __builtin_amdgcn_sched_barrier(0);
  }

  // ---- second product (bias in the start values), epilogue and stores per output tile
  const int rows = p.m - q0 < FF_P ? (int)(p.m - q0) : FF_P;
  const __amdgpu_buffer_rsrc_t orsrc = buf_rsrc_n((unsigned char*)p.out + q0 * RB, (uint32_t)(rows * RB));
#pragma unroll
  for (int T2 = 0; T2 < TG; ++T2) {
    // element j: channel 32 T2 + 16 (j / 8) + 8 hf + j % 8 = x fragment 2 T2 + j / 8, slot j % 8
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int ch = 32 * T2 + 16 * r + 8 * hf;
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(tab + 2 * C + ch);
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(tab + 2 * C + ch + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[8 * r + i] = b0[i];
        acc[8 * r + 4 + i] = b1[i];
      }
    }
#pragma unroll
    for (int T = 0; T < TG; ++T) {
      const unsigned char* wp = w2l + ((T2 * TG + T) * 64 + lane) * (16 * ES);
      if constexpr (DT == DT_BF16) {
        const bf16x8 w0 = *reinterpret_cast<const bf16x8*>(wp);
        const bf16x8 w1 = *reinterpret_cast<const bf16x8*>(wp + 16);
        acc = mfma32_bf16(w0, __builtin_bit_cast(bf16x8, uf[T][0]), acc);
        acc = mfma32_bf16(w1, __builtin_bit_cast(bf16x8, uf[T][1]), acc);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 w = *reinterpret_cast<const f32x4*>(wp + 16 * q);
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) acc = mfma32_f32(w[jj], uf[T][q][jj], acc);
        }
      }
    }
    float v[16];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int ch = 32 * T2 + 16 * r + 8 * hf;
      const f32x4 s0 = *reinterpret_cast<const f32x4*>(tab + 3 * C + ch);
      const f32x4 s1 = *reinterpret_cast<const f32x4*>(tab + 3 * C + ch + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[8 * r + i] = acc[8 * r + i] * s0[i] + xel<DT>(xr[2 * T2 + r], i);
        v[8 * r + 4 + i] = acc[8 * r + 4 + i] * s1[i] + xel<DT>(xr[2 * T2 + r], 4 + i);
      }
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int off = px * RB + (32 * T2 + 16 * r + 8 * hf) * ES;
      if constexpr (DT == DT_BF16) {
        u32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          o[i] = (unsigned)f32_to_bf16_bits(v[8 * r + 2 * i]) | ((unsigned)f32_to_bf16_bits(v[8 * r + 2 * i + 1]) << 16);
        __builtin_amdgcn_raw_buffer_store_b128(o, orsrc, off, 0, 0);
      } else {
        __builtin_amdgcn_raw_buffer_store_b128(
            __builtin_bit_cast(u32x4, f32x4{v[8 * r], v[8 * r + 1], v[8 * r + 2], v[8 * r + 3]}), orsrc, off, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b128(
            __builtin_bit_cast(u32x4, f32x4{v[8 * r + 4], v[8 * r + 5], v[8 * r + 6], v[8 * r + 7]}), orsrc,
            off + 16, 0, 0);
      }
    }
  }
}

template <int C, int DT, int PRO>
__global__ void __launch_bounds__(64 * ff_waves(C, DT)) ffn_kernel(const FfP p) {
  constexpr int NW = ff_waves(C, DT), D = ff_depth(C, DT), ES = ff_es(DT);
  constexpr int RB = C * ES;                 // bytes per pixel row
  constexpr int U = RB / 16;                 // 16-byte units per row
  constexpr int RPB = RB >= 256 ? 1 : 256 / RB;
  constexpr int UB = ff_unit_bytes(C, DT);
  constexpr int CP = UB / 1024;              // copy instructions per unit
  constexpr int KS = C / 16;                 // 16-k steps of the first product
  constexpr int TG = C / 32;                 // gated tiles = output tiles
  constexpr int W1B = 2 * C * C * ES, W2B = C * C * ES;
  constexpr int NS = TG * 2 * (ES / 2);      // 16-byte stores per lane per unit
  static_assert(UB % 1024 == 0 && (U & (U - 1)) == 0 && W1B % 1024 == 0 && W2B % 1024 == 0, "layout");
  static_assert((D - 2) * CP + (D - 1) * NS < 64, "vmcnt range");
  static_assert(PRO == PRO_NONE || PRO == PRO_LN || PRO == PRO_RMS, "prologue");
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  unsigned char* w1l = lds;
  unsigned char* w2l = lds + W1B;
  float* tab = reinterpret_cast<float*>(lds + W1B + W2B);  // b1 [2c] | b2 [c] | scale * out_scale [c]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: unit bases stay scalar
  const int px = lane & 31, hf = lane >> 5;
  unsigned char* ring = lds + ff_fixed_bytes(C, DT) + wave * (D * UB);

  // ---- packed weights -> LDS (both arrays are whole KiBs), tables
  for (int base = wave * 1024; base < W1B + W2B; base += NW * 1024) {
    const unsigned char* src = base < W1B ? (const unsigned char*)p.w1p + base
                                          : (const unsigned char*)p.w2p + (base - W1B);
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src + lane * 16),
                                     (__attribute__((address_space(3))) void*)(lds + base), 16, 0, 0);
  }
  for (int i = tid; i < 4 * C; i += 64 * NW) {
    float v;
    if (i < 2 * C) v = p.b1 ? p.b1[i] : 0.f;
    else if (i < 3 * C) v = p.b2 ? p.b2[i - 2 * C] : 0.f;
    else v = (p.scale ? p.scale[i - 3 * C] : 1.f) * p.out_scale;
    tab[i] = v;
  }

  const int nunits = (int)cdiv(p.m, FF_P);  // < 2^31 (checked by the host)
  const int stride = (int)gridDim.x * NW;
  const int wid = (int)blockIdx.x * NW + wave;
  const int nmine = wid < nunits ? (nunits - 1 - wid) / stride + 1 : 0;
  const unsigned char* X = (const unsigned char*)p.x;

  // copies of the wave's j-th unit into slot `slot` through a buffer bounded to the unit's valid
  // rows (rows past M read as zeros and are not stored); past the wave's last unit the last one
  // is copied again (never read), so every iteration issues CP copies
  auto issue = [&](int j, int slot) __attribute__((always_inline)) {
    const int unit = wid + (j < nmine ? j : nmine - 1) * stride;
    const int64_t q0 = (int64_t)unit * FF_P;
    const int rows = p.m - q0 < FF_P ? (int)(p.m - q0) : FF_P;
    const __amdgpu_buffer_rsrc_t r = buf_rsrc_n(X + q0 * RB, (uint32_t)(rows * RB));
    unsigned char* dst = ring + slot * UB;
#pragma unroll
    for (int c = 0; c < CP; ++c) {
      // byte offset in the unit of the 16 bytes this lane copies: LDS position (row, s) of a slot
      // holds the row's unit s ^ f(row)
      const int idx = c * 64 + lane;
      const int row = idx / U;
      const uint32_t off = row * RB + ff_swz(row, idx - row * U, U, RPB) * 16;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(dst + c * 1024), 16, off,
                                               0, 0, 0);
    }
  };

  // the lane's x fragments of the unit in `slot`: channels 16 s + 8 hf .. + 7 of pixel px
  auto read_frags = [&](int slot, typename XFragT<DT>::T (&xr)[KS]) __attribute__((always_inline)) {
    const unsigned char* xrow = ring + slot * UB + px * RB;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if constexpr (DT == DT_BF16) {
        xr[s] = *reinterpret_cast<const u32x4*>(xrow + ff_swz(px, 2 * s + hf, U, RPB) * 16);
      } else {
        const f32x4 a = *reinterpret_cast<const f32x4*>(xrow + ff_swz(px, 4 * s + 2 * hf, U, RPB) * 16);
        const f32x4 b = *reinterpret_cast<const f32x4*>(xrow + ff_swz(px, 4 * s + 2 * hf + 1, U, RPB) * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          xr[s].v[i] = a[i];
          xr[s].v[4 + i] = b[i];
        }
      }
    }
  };
  auto compute = [&](int j, int slot) __attribute__((always_inline)) {
    typename XFragT<DT>::T xr[KS];
    read_frags(slot, xr);
    ffn_unit<C, DT, PRO>(xr, w1l, w2l, tab, p, (int64_t)(wid + j * stride) * FF_P, lane);
  };

  // ---- the ring: units 0 .. D - 2 in flight before the first is computed, issued behind the
  // weight copies so that both travel together (the weights, issued first, have landed once at
  // most the (D - 1) x copy groups are outstanding). Iteration j issues the copies of unit j + D - 1
  // then unit j's NS stores, so when unit j is waited for, the operations issued after its copies
  // are (D - 2) copy groups and the stores of the last min(j, D - 1) units.
  if (nmine > 0) {
#pragma unroll
    for (int t = 0; t < D - 1; ++t) issue(t, t);
    wait_vmcnt<(D - 1) * CP>();
  } else {
    wait_vmem_all();
  }
  barrier_keep_vm();  // every wave's weight copies and table writes are in LDS
  if (nmine == 0) return;
  if constexpr (D == 1) {
    // one slot: unit j's fragments go to registers, then unit j + 1's copies refill the slot, so
    // when unit j + 1 is waited for only unit j's NS stores were issued after its copies
    issue(0, 0);
    for (int j = 0; j < nmine; ++j) {
      if (j > 0) wait_vmcnt<NS>();
      else wait_vmem_all();
      asm volatile("" ::: "memory");  // slot reads follow the wait
      typename XFragT<DT>::T xr[KS];
      read_frags(0, xr);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slot is free
      issue(j + 1, 0);
      ffn_unit<C, DT, PRO>(xr, w1l, w2l, tab, p, (int64_t)(wid + j * stride) * FF_P, lane);
    }
  } else {
    int sc = 0, si = D - 1;  // slots of the unit computed / issued in this iteration
    for (int j = 0; j < nmine; ++j) {
      if (j >= D - 1) wait_vmcnt<(D - 2) * CP + (D - 1) * NS>();
      else wait_vmcnt<(D - 2) * CP>();  // stricter than needed for j > 0
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // slot reads follow the wait; slot si is free
      issue(j + D - 1, si);
      compute(j, sc);
      sc = sc == D - 1 ? 0 : sc + 1;
      si = si == D - 1 ? 0 : si + 1;
    }
  }
  wait_vmem_all();
}

template <int C, int DT, int PRO>
void launch(const FfP& p, int nblk, hipStream_t s) {
  constexpr int lds = ff_lds_bytes(C, DT);
  auto fn = &ffn_kernel<C, DT, PRO>;
  static const bool attr = [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    return true;
  }();
  (void)attr;
  hipLaunchKernelGGL(fn, dim3((unsigned)nblk), dim3(64 * ff_waves(C, DT)), lds, s, p);
}

template <int C, int DT>
void launch_pro(const FfP& p, int pro, int nblk, hipStream_t s) {
  if (pro == PRO_LN) launch<C, DT, PRO_LN>(p, nblk, s);
  else if (pro == PRO_RMS) launch<C, DT, PRO_RMS>(p, nblk, s);
  else launch<C, DT, PRO_NONE>(p, nblk, s);
}

}  // namespace

}  // namespace clarus

using namespace clarus;

extern "C" int clarus_hip_ffn(const void* x, void* out, int dtype, const void* w1p, const float* b1, const void* w2p,
                              const float* b2, const float* scale, int64_t m, int64_t c, int pro, float ln_eps,
                              float out_scale, void* stream) {
  clear_error();
  CLARUS_REQUIRE(x && out && w1p && w2p, "ffn: null operand");
  CLARUS_REQUIRE(dtype == DT_BF16 || dtype == DT_F32, "ffn: bf16 or fp32 activations and weights");
  CLARUS_REQUIRE(c == 32 || c == 64 || (c == 128 && dtype == DT_BF16), "ffn: c = 32 or 64, or 128 in bf16 (c=%lld)",
                 (long long)c);
  CLARUS_REQUIRE(m > 0 && m < ((int64_t)1 << 35), "ffn: m out of range (m=%lld)", (long long)m);
  CLARUS_REQUIRE(pro == PRO_NONE || pro == PRO_LN || pro == PRO_RMS, "ffn: prologue none, LN or RMS");
  CLARUS_REQUIRE(aligned(x, 16) && aligned(out, 16) && aligned(w1p, 16) && aligned(w2p, 16),
                 "ffn: 16-byte aligned x, out and packed weights");
  const int64_t rb = c * ff_es(dtype);
  const char* xb = (const char*)x;
  const char* ob = (const char*)out;
  CLARUS_REQUIRE(ob + m * rb <= xb || xb + m * rb <= ob, "ffn: out must not overlap x");
  const int nw = dtype == DT_BF16 ? (c == 32 ? ff_waves(32, DT_BF16) : c == 64 ? ff_waves(64, DT_BF16)
                                                                            : ff_waves(128, DT_BF16))
                                  : (c == 32 ? ff_waves(32, DT_F32) : ff_waves(64, DT_F32));
  const int64_t units = cdiv(m, FF_P);
  int64_t nblk = device_cus();
  if (nblk > cdiv(units, nw)) nblk = cdiv(units, nw);
  FfP p{};
  p.x = x; p.w1p = w1p; p.w2p = w2p; p.b1 = b1; p.b2 = b2; p.scale = scale; p.out = out; p.m = m;
  p.ln_eps = ln_eps; p.out_scale = out_scale;
  note_kernel("ffn_kernel c=%lld dt=%s pro=%d", (long long)c, dtype == DT_BF16 ? "bf16" : "f32", pro);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == DT_BF16) {
    if (c == 32) launch_pro<32, DT_BF16>(p, pro, (int)nblk, s);
    else if (c == 64) launch_pro<64, DT_BF16>(p, pro, (int)nblk, s);
    else launch_pro<128, DT_BF16>(p, pro, (int)nblk, s);
  } else {
    if (c == 32) launch_pro<32, DT_F32>(p, pro, (int)nblk, s);
    else launch_pro<64, DT_F32>(p, pro, (int)nblk, s);
  }
  return check_launch("ffn");
}
