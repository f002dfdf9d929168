// Prologue passes of the long-K GEMMs: clarus_hip_rows_split and clarus_hip_rows_prologue.
//
// A GEMM whose A operand goes through a prologue (LayerNorm, RMS norm, the TLC local-mean map
// multiply) has fp32 values after the prologue, which bf16 MFMAs take as hi + lo bf16 pairs
// (|a - hi - lo| <= 2^-16 |a|). This pass applies the prologue to every row once and writes
// the pair as one bf16 row of 2K elements, [hi(0..K) | lo(0..K)]. The product with the
// duplicated weights [W | W] (2K rows of K-major W^T) is then an ordinary bf16 GEMM with
// K' = 2K, which runs on the DMA-pipelined 32x32-MFMA kernels instead of a register-staged
// prologue kernel. Prologue semantics: ops/torch_ref.py:94-100 (_ln, two-pass statistics, eps
// inside the square root), :85-91 and :18-41 (the TLC map expanded over the image with clamped
// coordinates), applied in fp32.
//
// Without a prologue (pro = none, fp32 rows) both passes only convert: the reference's fp32 A
// operand rounded to the bf16 weights' dtype before the product (kernels/gemm.py:187-193).
//
// clarus_hip_rows_prologue writes the prologue output rounded once to bf16 (RNE), a row of K
// elements, for a plain bf16 GEMM with the original K: the reference's GPU path for bf16 models
// (kernels/spatial.py:312 ln_rows with out_dtype = the compute dtype, :342 mul_small; used at
// ops/triton_cuda.py:104-110), which rounds the prologue output to the operand dtype before the
// tensor-core product (kernels/gemm.py:164, :175, :186).
//
// Work split: G lanes share a row (G = 16, 32 or 64, the power of two covering K / 8 up to 64),
// each holding FR fragments of 8 consecutive elements in registers; row statistics are exact
// two-pass sums over the group with a fixed butterfly order (bitwise reproducible). Stores are
// 16-byte vectors, contiguous across the group.
#include <algorithm>

#include "capi.hpp"
#include "gemm_kernel.hpp"

namespace clarus {

struct SplitP {
  const void* a;
  void* out;
  const void* small;
  int64_t m, k, lda;
  int pro, s_dt;
  int h, w, oh, ow, pt, pl;
  float eps;
};

template <int TA, int G, int FR, bool SPLIT>
__global__ void __launch_bounds__(256) rows_split_kernel(const SplitP p) {
  constexpr int ES = TA == DT_BF16 ? 2 : 4;
  constexpr int R = 64 / G;  // rows per wave
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / G, gl = lane - sub * G;
  const int64_t K = p.k;
  const float invk = 1.0f / (float)K;
  const int64_t step = (int64_t)gridDim.x * 4 * R;
  for (int64_t row = ((int64_t)blockIdx.x * 4 + wave) * R + sub; row < p.m; row += step) {
    const unsigned char* src = (const unsigned char*)p.a + row * p.lda * ES;
    f32x8 x[FR];
#pragma unroll
    for (int f = 0; f < FR; ++f) {
      const int64_t kk = (int64_t)(f * G + gl) * 8;
      x[f] = kk < K ? load8<TA>(src + kk * ES) : zero8();
    }
    if (p.pro == PRO_MUL) {  // a * S[clamp(y - pt), clamp(x - pl), k]
      const int hwi = p.h * p.w;
      const int64_t im = row / hwi;
      const int rr = (int)(row - im * hwi);
      const int yq = rr / p.w;
      int sy = yq - p.pt, sx = rr - yq * p.w - p.pl;
      sy = sy < 0 ? 0 : (sy > p.oh - 1 ? p.oh - 1 : sy);
      sx = sx < 0 ? 0 : (sx > p.ow - 1 ? p.ow - 1 : sx);
      const int64_t srow = ((im * p.oh + sy) * p.ow + sx) * K;
#pragma unroll
      for (int f = 0; f < FR; ++f) {
        const int64_t kk = (int64_t)(f * G + gl) * 8;
        if (kk >= K) continue;
        const f32x8 s = p.s_dt == DT_BF16 ? load8<DT_BF16>((const unsigned short*)p.small + srow + kk)
                                          : load8<DT_F32>((const float*)p.small + srow + kk);
#pragma unroll
        for (int i = 0; i < 8; ++i) x[f].v[i] *= s.v[i];
      }
    } else if (p.pro != PRO_NONE) {  // LayerNorm (two-pass mean / variance) or RMS norm
      float mean = 0.f;
      if (p.pro == PRO_LN) {
        float s = 0.f;
#pragma unroll
        for (int f = 0; f < FR; ++f)
#pragma unroll
          for (int i = 0; i < 8; ++i) s += x[f].v[i];
        mean = group_sum<G>(s) * invk;
      }
      float ss = 0.f;
#pragma unroll
      for (int f = 0; f < FR; ++f) {
        if ((int64_t)(f * G + gl) * 8 >= K) continue;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float d = x[f].v[i] - mean;
          ss += d * d;
        }
      }
      const float rstd = rsqrtf(group_sum<G>(ss) * invk + p.eps);
#pragma unroll
      for (int f = 0; f < FR; ++f)
#pragma unroll
        for (int i = 0; i < 8; ++i) x[f].v[i] = (x[f].v[i] - mean) * rstd;
    }
    unsigned short* dst = (unsigned short*)p.out + row * (SPLIT ? 2 : 1) * K;
#pragma unroll
    for (int f = 0; f < FR; ++f) {
      const int64_t kk = (int64_t)(f * G + gl) * 8;
      if (kk >= K) continue;
      if constexpr (SPLIT) {
        bf16x8 hi, lo;
        split_bf16(x[f], hi, lo);
        *reinterpret_cast<bf16x8*>(dst + kk) = hi;
        *reinterpret_cast<bf16x8*>(dst + K + kk) = lo;
      } else {
        *reinterpret_cast<bf16x8*>(dst + kk) = pack_bf16(x[f]);
      }
    }
  }
}

template <int TA, int G, int FR, bool SPLIT>
static void launch_split(const SplitP& p, hipStream_t s) {
  constexpr int rows_per_block = 4 * (64 / G);
  const unsigned blocks = (unsigned)std::min<int64_t>(cdiv(p.m, rows_per_block), 4096);
  note_kernel("rows_split_kernel g=%d split=%d", G, (int)SPLIT);
  hipLaunchKernelGGL((rows_split_kernel<TA, G, FR, SPLIT>), dim3(blocks), dim3(256), 0, s, p);
}

template <int TA, bool SPLIT>
static void launch_split_ta(const SplitP& p, hipStream_t s) {
  const int64_t frags = p.k / 8;  // 8-element fragments per row
  if (frags <= 16) launch_split<TA, 16, 1, SPLIT>(p, s);
  else if (frags <= 32) launch_split<TA, 32, 1, SPLIT>(p, s);
  else if (frags <= 64) launch_split<TA, 64, 1, SPLIT>(p, s);
  else if (frags <= 128) launch_split<TA, 64, 2, SPLIT>(p, s);
  else launch_split<TA, 64, 4, SPLIT>(p, s);
}

// shared argument checks and launch of both entry points
static int rows_pass(const ClarusGemmArgs* a, void* out, void* stream, bool split, const char* what) {
  clear_error();
  CLARUS_REQUIRE(a != nullptr && a->a && out, "%s: null operand", what);
  CLARUS_REQUIRE(a->m > 0 && a->k > 0, "%s: empty problem", what);
  CLARUS_REQUIRE(a->pro == PRO_NONE || a->pro == PRO_LN || a->pro == PRO_RMS || a->pro == PRO_MUL,
                 "%s: prologue %d is not none, LN, RMS or the map multiply", what, a->pro);
  CLARUS_REQUIRE(a->pro != PRO_NONE || a->a_dtype == DT_F32, "%s: rows without a prologue must be fp32", what);
  CLARUS_REQUIRE(a->a_dtype == DT_F32 || a->a_dtype == DT_BF16, "%s: bad A dtype", what);
  CLARUS_REQUIRE(a->k % 8 == 0 && a->k <= 2048, "%s: K=%lld must be a multiple of 8, at most 2048", what,
                 (long long)a->k);
  const int ea = a->a_dtype == DT_BF16 ? 2 : 4;
  CLARUS_REQUIRE(aligned(a->a, 16) && aligned(out, 16) && (a->lda * ea) % 16 == 0 && a->lda >= a->k,
                 "%s: A rows and the output must be 16-byte aligned", what);
  CLARUS_REQUIRE(a->batch == 1, "%s: rows of one batch entry (fold images into m)", what);
  if (a->pro == PRO_MUL) {
    CLARUS_REQUIRE(a->small && (a->s_dtype == DT_F32 || a->s_dtype == DT_BF16) && aligned(a->small, 16),
                   "%s: the map multiply needs an aligned map", what);
    CLARUS_REQUIRE(a->h > 0 && a->w > 0 && a->oh > 0 && a->ow > 0 && a->m % ((int64_t)a->h * a->w) == 0,
                   "%s: map geometry", what);
  }
  SplitP p{};
  p.a = a->a; p.out = out; p.small = a->small;
  p.m = a->m; p.k = a->k; p.lda = a->lda;
  p.pro = a->pro; p.s_dt = a->s_dtype;
  p.h = a->h; p.w = a->w; p.oh = a->oh; p.ow = a->ow; p.pt = a->pt; p.pl = a->pl;
  p.eps = a->ln_eps;
  hipStream_t s = (hipStream_t)stream;
  if (a->a_dtype == DT_BF16) split ? launch_split_ta<DT_BF16, true>(p, s) : launch_split_ta<DT_BF16, false>(p, s);
  else split ? launch_split_ta<DT_F32, true>(p, s) : launch_split_ta<DT_F32, false>(p, s);
  return check_launch(what);
}

}  // namespace clarus

using namespace clarus;

extern "C" int clarus_hip_rows_split(const ClarusGemmArgs* a, void* out, void* stream) {
  return rows_pass(a, out, stream, true, "rows_split");
}

extern "C" int clarus_hip_rows_prologue(const ClarusGemmArgs* a, void* out, void* stream) {
  return rows_pass(a, out, stream, false, "rows_prologue");
}
