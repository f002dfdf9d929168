// C entry points of the fused GEMM family: clarus_hip_gemm, clarus_hip_conv3x3,
// clarus_hip_intro3x3. Argument checks happen here, before any launch.
#include <algorithm>

#include "capi.hpp"
#include "gemm_dispatch.hpp"
#include "gemm_lds_dispatch.hpp"
#include "gemm_stream_dispatch.hpp"
#include "gemm_rowstream_dispatch.hpp"

namespace clarus {

static int esize(int dt) { return dt == DT_BF16 ? 2 : 4; }
static bool dt_ok(int dt) { return dt == DT_F32 || dt == DT_BF16; }

// widest vector access that keeps every channel run aligned: 2 = 16 B, 1 = 8 B / quad, 0 = scalar
static int vec_level(const void* base, int es, int64_t ld, int64_t bstride) {
  auto ok = [&](int bytes) {
    return aligned(base, bytes) && (ld * es) % bytes == 0 && (bstride * es) % bytes == 0;
  };
  if (ok(16)) return 2;
  if (ok(4 * es)) return 1;
  return 0;
}

static int operand_mode(int a_dt, int w_dt, bool transformed) {
  if (w_dt == DT_F32) return OPM_F32;
  if (a_dt == DT_BF16 && !transformed) return OPM_BF16;
  return OPM_SPLIT;
}

// tile id for a problem: channel tile from n, pixel tile from the amount of parallel work.
// run_div: the lane's channel run (4 * NB) must divide it (pixel-shuffle quadrant width), 0 = any
static int auto_tile(int64_t m, int64_t n, int64_t k, int64_t batch, bool gate, int opm, int64_t run_div) {
  int t;
  if (n <= 16) t = 0;
  else if (n <= 32) t = 1;
  else if (n <= 64 || gate || opm == OPM_F32 || k > kc_for(opm)) t = 3;
  else t = 6;
  while (run_div && (run_div % (4 * kTileNB[t])) != 0) t = (kTileNB[t] == 8) ? 3 : (kTileNB[t] == 4 ? 1 : 0);
  const int64_t tn = 16 * kTileNB[t];
  const int64_t wgs = cdiv(m, 64 * kTilePB[t]) * cdiv(n, tn) * batch;
  if (wgs < 1024) {
    if (t == 3) t = 2;
    if (t == 6) t = 5;
  }
  return t;
}

// persistent grid: when W^T fits in one LDS chunk a workgroup keeps it and walks several
// pixel tiles; aim for ~4 resident workgroups per CU
static dim3 grid_for(int64_t ptiles, int64_t ntiles, int64_t batch, int64_t k, int kc) {
  int64_t gx = ptiles;
  if (k <= kc) {
    const int64_t target = 4LL * device_cus();
    int64_t per = ntiles * batch;
    int64_t want = (target + per - 1) / per;
    if (want < 1) want = 1;
    if (want < ptiles) {
      const int64_t tiles_per = cdiv(ptiles, want);
      gx = cdiv(ptiles, tiles_per);
    }
  }
  return dim3((unsigned)gx, (unsigned)ntiles, (unsigned)batch);
}

// ------------------------------------------------------------------- LayerNorm / RMS statistics
// One wave per row (persistent over rows): the row is read once into registers (up to 2048
// elements; longer rows are re-read for the second pass), exact two-pass mean and variance,
// wave-wide butterfly sums (fixed order, deterministic). stats[2 r] = mean (0 for RMS),
// stats[2 r + 1] = rsqrt(var + eps) (rsqrt(mean(x^2) + eps) for RMS).
// Semantics of kernels/gemm.py:289-313 row_stats / ops/torch_ref.py:94-100.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <int TA>
__global__ void __launch_bounds__(256) row_stats_kernel(const void* a, int64_t lda, int64_t m, int64_t k, int rms,
                                                        float eps, float* stats) {
  constexpr int ES = TA == DT_BF16 ? 2 : 4;
  constexpr int CACHED = 4;  // fragments of 8 per lane kept in registers (K <= 2048)
  const int lane = threadIdx.x & 63;
  const float invk = 1.0f / (float)k;
  for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < m; row += (int64_t)gridDim.x * 4) {
    const unsigned char* base = (const unsigned char*)a + row * lda * ES;
    f32x8 x[CACHED];
#pragma unroll
    for (int j = 0; j < CACHED; ++j) {
      const int64_t kk = (int64_t)(j * 64 + lane) * 8;
      x[j] = kk < k ? load8<TA>(base + kk * ES) : zero8();
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < CACHED; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) s += x[j].v[i];
    for (int64_t kk = (int64_t)(CACHED * 64 + lane) * 8; kk < k; kk += 512) {
      const f32x8 t = load8<TA>(base + kk * ES);
#pragma unroll
      for (int i = 0; i < 8; ++i) s += t.v[i];
    }
    const float mean = rms ? 0.f : wave_sum(s) * invk;
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < CACHED; ++j) {
      if ((int64_t)(j * 64 + lane) * 8 >= k) continue;
#pragma unroll
      for (int i = 0; i < 8; ++i) { const float d = x[j].v[i] - mean; ss += d * d; }
    }
    for (int64_t kk = (int64_t)(CACHED * 64 + lane) * 8; kk < k; kk += 512) {
      const f32x8 t = load8<TA>(base + kk * ES);
#pragma unroll
      for (int i = 0; i < 8; ++i) { const float d = t.v[i] - mean; ss += d * d; }
    }
    const float rstd = rsqrtf(wave_sum(ss) * invk + eps);
    if (lane == 0) *reinterpret_cast<f32x2*>(stats + 2 * row) = f32x2{mean, rstd};
  }
}

static void launch_row_stats(const void* a, int a_dt, int64_t lda, int64_t m, int64_t k, bool rms, float eps,
                             float* stats, hipStream_t s) {
  const unsigned blocks = (unsigned)std::min<int64_t>(cdiv(m, 4), 8LL * device_cus());
  if (a_dt == DT_BF16)
    hipLaunchKernelGGL(row_stats_kernel<DT_BF16>, dim3(blocks), dim3(256), 0, s, a, lda, m, k, (int)rms, eps, stats);
  else
    hipLaunchKernelGGL(row_stats_kernel<DT_F32>, dim3(blocks), dim3(256), 0, s, a, lda, m, k, (int)rms, eps, stats);
}

static int launch(GemmP& p, int am, bool gate, int opm, int ta, int tile, int64_t batch,
                  hipStream_t s, const char* what) {
  if (tile < 0 || tile >= kNumTiles) {
    set_error("%s: tile id %d out of range", what, tile + 1);
    return CLARUS_EINVAL;
  }
  GemmLaunch fn = nullptr;
  if (am == AM_ROWS) fn = pick_gemm_rows(tile, gate, opm, ta);
  else if (am == AM_S2D) fn = pick_gemm_s2d(tile, opm, ta);
  else fn = pick_gemm_conv(tile, opm, ta);
  if (!fn) {
    set_error("%s: no kernel for tile %d gate %d operand mode %d A dtype %d", what, tile, (int)gate,
              opm, ta);
    return CLARUS_EINVAL;
  }
  const int64_t tn = 16 * kTileNB[tile];
  const int64_t tp = 64 * kTilePB[tile];
  p.ptiles = cdiv(p.m, tp);
  dim3 g = grid_for(p.ptiles, cdiv(p.n, tn), batch, p.k, kc_for(opm));
  fn(p, g, s, p.k <= kc_for(opm) ? 1 : 2);
  return check_launch(what);
}

}  // namespace clarus

using namespace clarus;

extern "C" int clarus_hip_gemm(const ClarusGemmArgs* a, void* stream) {
  clear_error();
  CLARUS_REQUIRE(a != nullptr, "gemm: null args");
  // CLARUS_PRO_ROUND: the prologue output may be rounded once to bf16 (the ring streaming
  // kernel does; the other kernels keep hi + lo pairs)
  ClarusGemmArgs plain;
  const bool pro_round = (a->pro & CLARUS_PRO_ROUND) != 0;
  if (pro_round) {
    plain = *a;
    plain.pro &= ~CLARUS_PRO_ROUND;
    a = &plain;
  }
  CLARUS_REQUIRE(a->a && a->wt && a->c, "gemm: null operand");
  CLARUS_REQUIRE(a->m > 0 && a->n > 0 && a->k > 0 && a->batch > 0, "gemm: empty problem m=%lld n=%lld k=%lld",
                 (long long)a->m, (long long)a->n, (long long)a->k);
  CLARUS_REQUIRE(dt_ok(a->a_dtype) && dt_ok(a->w_dtype) && dt_ok(a->c_dtype), "gemm: bad dtype code");
  CLARUS_REQUIRE(a->k % 8 == 0, "gemm: K=%lld must be a multiple of 8", (long long)a->k);
  CLARUS_REQUIRE(a->a_mode == CLARUS_A_ROWS || a->a_mode == CLARUS_A_S2D, "gemm: bad a_mode %d", a->a_mode);
  CLARUS_REQUIRE(a->c_mode == CLARUS_C_ROWS || a->c_mode == CLARUS_C_SHUFFLE, "gemm: bad c_mode %d", a->c_mode);
  CLARUS_REQUIRE(a->pro == PRO_NONE || a->pro == PRO_LN || a->pro == PRO_MUL || a->pro == PRO_RMS ||
                     a->pro == PRO_LNMUL, "gemm: bad prologue %d", a->pro);
  CLARUS_REQUIRE(a->act == ACT_NONE || a->act == ACT_GELU || a->act == ACT_LRELU, "gemm: bad act %d", a->act);
  CLARUS_REQUIRE(!(a->gate && a->a_mode != CLARUS_A_ROWS), "gemm: gate only with row operands");
  CLARUS_REQUIRE(a->a_mode == CLARUS_A_ROWS || a->pro == PRO_NONE, "gemm: prologues only with row operands");
  const int ea = esize(a->a_dtype), ew = esize(a->w_dtype);
  CLARUS_REQUIRE(aligned(a->a, 16) && aligned(a->wt, 16), "gemm: A and W must be 16-byte aligned");
  CLARUS_REQUIRE(a->batch == 1 || (a->a_bstride * ea) % 16 == 0, "gemm: A batch stride alignment");
  CLARUS_REQUIRE(a->batch == 1 || (a->w_bstride * ew) % 16 == 0, "gemm: W batch stride alignment");

  GemmP p{};
  p.a = a->a; p.wt = a->wt; p.c = a->c;
  p.bias = a->bias; p.scale = a->scale; p.res = a->res;
  p.small = a->small; p.m2 = a->m2; p.lnw = a->lnw; p.lnb = a->lnb;
  p.stats = nullptr;
  p.m = a->m; p.n = a->n; p.k = a->k;
  p.lda = a->lda; p.ldc = a->ldc; p.ldr = a->ldr; p.ldm2 = a->ldm2;
  p.a_bs = a->a_bstride; p.w_bs = a->w_bstride; p.c_bs = a->c_bstride; p.r_bs = a->r_bstride;
  p.c_dt = a->c_dtype; p.r_dt = a->r_dtype; p.s_dt = a->s_dtype; p.m2_dt = a->m2_dtype;
  p.h = a->h; p.w = a->w; p.oh = a->oh; p.ow = a->ow; p.pt = a->pt; p.pl = a->pl;
  p.pro = a->pro; p.c_mode = a->c_mode; p.act = a->act; p.m2_act = a->m2_act;
  p.has_res = a->res != nullptr;
  p.ln_eps = a->ln_eps; p.out_scale = a->out_scale; p.slope = a->slope;
  p.up2 = 0;

  if (a->a_mode == CLARUS_A_ROWS) {
    CLARUS_REQUIRE((a->lda * ea) % 16 == 0 && a->lda >= a->k, "gemm: lda=%lld must cover K and keep 16-byte rows",
                   (long long)a->lda);
  } else {
    CLARUS_REQUIRE(a->k % 32 == 0, "gemm: space-to-depth needs K = 4 * cin with cin %% 8 == 0");
    CLARUS_REQUIRE(a->h > 1 && a->w > 1, "gemm: space-to-depth needs h, w >= 2");
    CLARUS_REQUIRE(a->m % ((int64_t)(a->h / 2) * (a->w / 2)) == 0 && a->batch == 1,
                   "gemm: space-to-depth rows must be whole output images");
    p.cin = (int)(a->k / 4);
    p.lda = p.cin;
  }
  if (a->pro == PRO_MUL) {
    CLARUS_REQUIRE(a->small && dt_ok(a->s_dtype) && aligned(a->small, 16), "gemm: mul prologue needs an aligned map");
    CLARUS_REQUIRE(a->h > 0 && a->w > 0 && a->oh > 0 && a->ow > 0 && a->m % ((int64_t)a->h * a->w) == 0 &&
                       a->batch == 1, "gemm: mul prologue geometry");
  }
  if (a->pro == PRO_LNMUL) {
    CLARUS_REQUIRE(a->m2 && a->lnw && a->lnb && dt_ok(a->m2_dtype), "gemm: LN-mul prologue operands");
    CLARUS_REQUIRE(aligned(a->m2, 16) && (a->ldm2 * esize(a->m2_dtype)) % 16 == 0 && aligned(a->lnw, 16) &&
                       aligned(a->lnb, 16) && a->batch == 1, "gemm: LN-mul operand alignment");
  }
  if (a->res) CLARUS_REQUIRE(dt_ok(a->r_dtype), "gemm: bad residual dtype");
  const int ec = esize(a->c_dtype);
  if (a->c_mode == CLARUS_C_SHUFFLE) {
    CLARUS_REQUIRE(a->n % 16 == 0 && a->h > 0 && a->w > 0 && a->m % ((int64_t)a->h * a->w) == 0 && a->batch == 1,
                   "gemm: pixel-shuffle output needs N %% 16 == 0 and whole images");
    p.vec_out = vec_level(a->c, ec, 0, 0);
    p.vec_res = a->res ? vec_level(a->res, esize(a->r_dtype), 0, 0) : 0;
  } else {
    CLARUS_REQUIRE(a->ldc >= a->n, "gemm: ldc < n");
    p.vec_out = vec_level(a->c, ec, a->ldc, a->c_bstride);
    p.vec_res = a->res ? vec_level(a->res, esize(a->r_dtype), a->ldr, a->r_bstride) : 0;
  }

  const bool transformed = a->pro != PRO_NONE;
  const int opm = operand_mode(a->a_dtype, a->w_dtype, transformed);
  const int64_t run_div = a->c_mode == CLARUS_C_SHUFFLE ? a->n / 4 : 0;
  // W-resident streaming kernel for row operands with K <= 256 (bf16 A) / 128 (fp32 A) (tile 0 = auto, 8 / 9 = force
  // NB 4 / 8); the tiled kernel otherwise (tiles 1..7 force one of its tile shapes)
  // Automatic choice for bf16 rows without a prologue (measured on the config-2 shapes):
  // K > 128 (K % 32 == 0): the DMA-pipelined tile kernel; K <= 128 with a residual: the tiled
  // kernel with 64 x 64 tiles (the streaming kernel's residual prefetch costs it ~25 % there).
  const bool plain_bf16 = a->a_mode == CLARUS_A_ROWS && opm == OPM_BF16 && a->pro == PRO_NONE && a->batch == 1;
  // few 128 x 128 output tiles (under 192 for 256 CUs): the 64 x 64 tiled kernel fills the GPU
  // better (NAFNet SCA GEMMs on the TLC map: M = 4859, K = N = 512: 15.9 vs 17.2 us; M = 1254,
  // K = N = 1024: 20.0 vs 24.0 us; c1024 c -> c with 232 tiles stays: 30.8 vs 28.3 us)
  const bool few_tiles = a->tile == 0 && plain_bf16 && a->k > 128 && !run_div &&
                         cdiv(a->m, 128) * cdiv(a->n, a->gate ? 64 : 128) < 192;
  const bool auto_dma = a->tile == 0 && plain_bf16 && a->k > 128 && a->k % 32 == 0 && (a->lda * 2) % 16 == 0 &&
                        (!run_div || run_div % gemm_lds_run(a->gate != 0) == 0) && !few_tiles;
  // W-slice kernel (tile 18 forces it): plain problems without residual, gate or activation and
  // up to 80 K rows (the NAFNet SCA GEMMs on the TLC map, us, HIP events, cold / warm:
  // M = 4859, K = N = 512: 12.8 / 11.2 against 17.0 / 15.4 on the DMA tile kernel and 15.8 / 13.6
  // on the weight-streaming one; 19125 x 256: 14.0 / 12.1 vs 15.6 / 13.7 (W-resident kernel);
  // 75881 x 128: 16.0 / 12.9 vs 17.4 / 16.4 (streaming kernel))
  {
    const bool slice_shape = plain_bf16 && !a->gate && !a->res && a->act == ACT_NONE &&
                             a->c_mode == CLARUS_C_ROWS && gemm_slice_fits(p);
    CLARUS_REQUIRE(a->tile != 18 || slice_shape, "gemm: the W-slice kernel does not take this problem");
    if (a->tile == 18 || (a->tile == 0 && slice_shape && a->m <= 80000)) {
      note_kernel("gemm_slice_kernel k=%lld c=%s", (long long)a->k, a->c_dtype == DT_BF16 ? "bf16" : "f32");
      CLARUS_REQUIRE(launch_gemm_slice(p, (hipStream_t)stream), "gemm: W-slice launch");
      return check_launch("gemm");
    }
  }
  int tile_override = 0;
  if (a->tile == 0 && plain_bf16 && a->res && a->k <= 128 && (!run_div || run_div % 16 == 0)) tile_override = 3;
  if (few_tiles) tile_override = 3;
  // streaming kernel with an LDS ring per wave: rows without prologue or with LN / RMS / a bf16
  // TLC map (split operands, batch 1), row or pixel-shuffle output (a lane's channel run inside
  // one quadrant), K <= 128 (bf16 A) / 64 (fp32 A); a residual needs 16-byte rows and whole
  // 16-byte channel units, and no gate. Automatic for K <= 64 and for K <= 128 without a gate (measured against the
  // register-prefetch streaming kernel and the 64 x 64 tiled kernel on the NAFNet, config-1 and
  // attn . V shapes: faster or equal except a gated K = 128); tile 16 forces it.
  {
    const int ks = rowstream_ks_for(a->k, a->a_dtype);
    const int er = a->res ? esize(a->r_dtype) : 2;
    const bool res_ok = !a->res || (p.vec_res == 2 && a->n % (16 / er) == 0 && !a->gate);
    const int nb = (a->n <= 64 || a->gate || a->tile == 17) ? 4 : (run_div && run_div % 32 ? 4 : 8);
    const bool pro_ok = a->pro == PRO_NONE ||
                        (opm == OPM_SPLIT && a->batch == 1 &&
                         (a->pro == PRO_LN || a->pro == PRO_RMS || (a->pro == PRO_MUL && a->s_dtype == DT_BF16)));
    const bool ring_ok = a->a_mode == CLARUS_A_ROWS && pro_ok && ks && res_ok &&
                         (opm != OPM_SPLIT || a->a_dtype == DT_F32 || a->pro != PRO_NONE) &&
                         (!run_div || (run_div % (4 * nb) == 0 && a->batch == 1));
    CLARUS_REQUIRE((a->tile != 16 && a->tile != 17) || ring_ok,
                   "gemm: the ring streaming kernel does not take this problem");
    // K = 128 (interleaved A/B on the NAFNet shapes, us): a row-layout residual takes the ring
    // with 4 channel blocks (c128 c->c 37.0 vs 41.3 on the 64 x 64 tiles, 45.0 with 8 blocks);
    // a pixel-shuffled residual the 64 x 64 tiles (level-1 -> 0 up-conv 76 vs 109); a gate the
    // register-prefetch streaming kernel (36.6 vs 38.6); neither the streaming kernel with 4
    // channel blocks (level-1 conv1 46.9 vs 50.9)
    const bool ring_res128 = a->tile == 0 && ring_ok && ks == 4 && a->res && !run_div && !a->gate;
    const bool ring_auto = a->tile == 0 && ring_ok && (ks <= 2 || ring_res128);
    const int rnb = (a->tile == 17 || ring_res128) ? 4 : nb;
    if (a->tile == 16 || a->tile == 17 || ring_auto) {
      GemmP q = p;
      q.ptiles = 0;
      // 8 channel blocks when the ring still fits next to W^T, else 4
      const int ropm = (pro_round && opm == OPM_SPLIT && a->a_dtype == DT_BF16 && a->pro != PRO_NONE) ? OPM_ROUND : opm;
      note_kernel("gemm_rowstream_kernel nb=%d gate=%d opm=%d ks=%d res=%d", rnb, a->gate != 0, ropm, ks,
                  a->res != nullptr);
      if (launch_gemm_rowstream(q, rnb, a->gate != 0, ropm, a->a_dtype, ks, a->res != nullptr, a->r_dtype, a->batch,
                                (hipStream_t)stream) ||
          (rnb == 8 && (note_kernel("gemm_rowstream_kernel nb=4 gate=%d opm=%d ks=%d res=%d", a->gate != 0, ropm,
                                    ks, a->res != nullptr),
                        launch_gemm_rowstream(q, 4, a->gate != 0, ropm, a->a_dtype, ks, a->res != nullptr, a->r_dtype,
                                              a->batch, (hipStream_t)stream))))
        return check_launch("gemm");
      CLARUS_REQUIRE(a->tile == 0, "gemm: no ring streaming kernel for operand mode %d A dtype %d K=%lld", opm,
                     a->a_dtype, (long long)a->k);
    }
  }
  // fp32 weights stream with fp32 A and K <= 128, no second prologue operand (LDS holds fp32 rows)
  const bool stream_opm = opm != OPM_F32 || (a->a_dtype == DT_F32 && a->pro != PRO_MUL && a->pro != PRO_LNMUL);
  if (a->a_mode == CLARUS_A_ROWS && stream_opm && !auto_dma && !tile_override &&
      (a->tile == 0 || a->tile == 8 || a->tile == 9)) {
    const int ks = stream_ks_for(a->k, a->a_dtype);
    int nb = a->tile == 8 ? 4 : a->tile == 9 ? 8 : ((a->n <= 64 || a->gate || a->k > 64) ? 4 : 8);
    if (opm == OPM_F32 && a->gate) nb = 4;  // fp32 gate rows of NB 8 exceed the LDS budget
    if (run_div && run_div % (4 * nb)) nb = 4;
    const bool x2 = a->pro == PRO_MUL || a->pro == PRO_LNMUL;
    GemmLaunch fn = (ks && (!run_div || run_div % (4 * nb) == 0)) ? pick_gemm_stream(nb, a->gate != 0, opm, a->a_dtype, ks, x2)
                                                                : nullptr;
    if (fn) {
      p.ptiles = 0;
      note_kernel("gemm_stream_kernel nb=%d gate=%d opm=%d ks=%d", nb, a->gate != 0, opm, ks);
      fn(p, dim3(0, (unsigned)cdiv(a->n, 16 * nb), (unsigned)a->batch), (hipStream_t)stream, 1);
      return check_launch("gemm");
    }
    CLARUS_REQUIRE(a->tile == 0, "gemm: no streaming kernel for K=%lld nb=%d", (long long)a->k, nb);
  }
  // pipelined LDS-tiled kernel for long-K row operands (tile 0 = auto for K > 128, 10 = force);
  // LN-type prologues need the statistics scratch there
  const bool ln_like = a->pro == PRO_LN || a->pro == PRO_RMS || a->pro == PRO_LNMUL;
  const bool lds_shape = a->a_mode == CLARUS_A_ROWS && opm != OPM_F32 && a->batch == 1 &&
                         (!run_div || run_div % gemm_lds_run(a->gate != 0) == 0);
  const bool use_lds = lds_shape && (a->tile == 10 || (a->tile == 0 && a->k > 128 && !few_tiles)) &&
                       (!ln_like || a->stats);
  CLARUS_REQUIRE(a->tile != 10 || use_lds, "gemm: the pipelined tile kernel does not take this problem");
  const bool needs_stats = a->a_mode == CLARUS_A_ROWS && ln_like && (use_lds || a->k > kc_for(opm));
  if (needs_stats && a->stats && a->batch == 1) {  // one pass over A instead of one per column tile
    CLARUS_REQUIRE(aligned(a->stats, 8), "gemm: stats scratch must be 8-byte aligned");
    launch_row_stats(a->a, a->a_dtype, a->lda, a->m, a->k, a->pro == PRO_RMS, a->ln_eps, a->stats,
                     (hipStream_t)stream);
    p.stats = a->stats;
  }
  // bf16 operands without prologue: the DMA-pipelined kernels. K % 64 == 0 runs on 32x32x16
  // MFMAs with 64-k chunks (tile 13 forces it), other K % 32 == 0 on 16x16x32 MFMAs with 32-k
  // chunks (tile 11 forces it)
  const bool dma_ok = lds_shape && opm == OPM_BF16 && a->pro == PRO_NONE && a->k % 32 == 0 &&
                      (a->lda * 2) % 16 == 0 &&
                      cdiv(a->m, 128) * cdiv(a->n, 64) < ((int64_t)1 << 31);  // tile index in 31 bits
  const bool m32_ok = dma_ok && a->k % 64 == 0 && (!run_div || run_div % kGemmM32Run == 0) &&
                      epi32_tables_fit(a->n, a->gate != 0);  // bias / scale tables in LDS
  // 2x2 stride-2 down conv with bf16 operands: space-to-depth rows on the 32x32 DMA-pipelined
  // kernel (tile 13 or auto; tiles 1-7 keep the register-staged tiled kernel)
  const bool s2d_m32 = a->a_mode == CLARUS_A_S2D && opm == OPM_BF16 && a->pro == PRO_NONE && a->batch == 1 &&
                       p.cin % 32 == 0 && !run_div && epi32_tables_fit(a->n, a->gate != 0) &&
                       cdiv(a->m, 128) * cdiv(a->n, 64) < ((int64_t)1 << 31);
  CLARUS_REQUIRE(a->tile != 11 || dma_ok, "gemm: the DMA-pipelined kernel does not take this problem");
  CLARUS_REQUIRE(a->tile != 13 || m32_ok || s2d_m32,
                 "gemm: the 32x32 DMA-pipelined kernel does not take this problem");
  if (s2d_m32 && (a->tile == 0 || a->tile == 13)) {
    p.s2d = 1;
    note_kernel("gemm_mfma32_kernel s2d=1 gate=%d", a->gate != 0);
    launch_gemm_m32(p, a->gate != 0, (hipStream_t)stream);
    return check_launch("gemm");
  }
  CLARUS_REQUIRE((a->tile != 14 && a->tile != 15) || m32_ok,
                 "gemm: the big-tile DMA-pipelined kernel does not take this problem");
  // Automatic choice among the DMA-pipelined kernels for plain bf16 rows with K > 128
  // (interleaved A/B on the NAFNet shapes, us):
  //   * gated, with at least 200 tiles of 256 pixels x 256 W^T rows: gemm_big_kernel (level-3
  //     conv4 28.8 vs 31.7 on 32x32 / 29.8 on 16x16; level-2 conv4 33.6 vs 37.4 / 35.9);
  //   * with a residual, K > 256 and at least 320 tiles of 128 x 128: 32x32 MFMAs (K = 512 with an
  //     fp32 residual, 452 tiles: 25.2 vs 28.6); with fewer tiles 16x16 (config-2 c1024
  //     c->c+scale+res, 3600 x 1024 x 1024, 232 tiles: 29.3 vs 32.1);
  //   * otherwise 16x16 MFMAs (level-3 conv1 34.0 vs 36.7; level-2 conv1 41.6 vs 43.8;
  //     c1024 rows 29.1 vs 32.1; c256 c->c+scale+res 31.2 vs 35.6)
  const bool long_auto = a->tile == 0 && (auto_dma || use_lds);
  const bool big_auto = long_auto && m32_ok && a->gate && !a->res && cdiv(a->m, 256) * cdiv(a->n, 128) >= 200;
  if (a->tile == 14 || a->tile == 15 || big_auto) {
    note_kernel("gemm_big_kernel gate=%d wp=%d", a->gate != 0, a->tile == 15 ? 1 : 2);
    launch_gemm_big(p, a->gate != 0, a->tile == 15 ? 1 : 2, (hipStream_t)stream);
    return check_launch("gemm");
  }
  const bool m32_auto = m32_ok && long_auto && a->res && a->k > 256 && cdiv(a->m, 128) * cdiv(a->n, 128) >= 320;
  if (a->tile == 13 || m32_auto) {
    note_kernel("gemm_mfma32_kernel gate=%d", a->gate != 0);
    launch_gemm_m32(p, a->gate != 0, (hipStream_t)stream);
    return check_launch("gemm");
  }
  if (dma_ok && (a->tile == 11 || auto_dma || (use_lds && a->tile == 0))) {
    note_kernel("gemm_dma_kernel gate=%d", a->gate != 0);
    launch_gemm_dma(p, a->gate != 0, (hipStream_t)stream);
    return check_launch("gemm");
  }
  if (use_lds) {
    const bool x2 = a->pro == PRO_MUL || a->pro == PRO_LNMUL;
    note_kernel("gemm_lds_kernel gate=%d opm=%d x2=%d", a->gate != 0, opm, x2);
    CLARUS_REQUIRE(launch_gemm_lds(p, a->gate != 0, opm, a->a_dtype, x2, (hipStream_t)stream),
                   "gemm: no pipelined tile kernel for operand mode %d A dtype %d", opm, a->a_dtype);
    return check_launch("gemm");
  }
  const int tile = a->tile > 0 ? a->tile - 1
                   : tile_override ? tile_override - 1
                                   : auto_tile(a->m, a->n, a->k, a->batch, a->gate != 0, opm, run_div);
  CLARUS_REQUIRE(tile >= 0 && tile < kNumTiles && (!run_div || run_div % (4 * kTileNB[tile]) == 0),
                 "gemm: tile %d does not fit the pixel-shuffle quadrant width", tile + 1);
  note_kernel("gemm_kernel tile=%d am=%s gate=%d opm=%d", tile + 1, a->a_mode == CLARUS_A_ROWS ? "rows" : "s2d",
              a->gate != 0, opm);
  return launch(p, a->a_mode == CLARUS_A_ROWS ? AM_ROWS : AM_S2D, a->gate != 0, opm, a->a_dtype, tile, a->batch,
                (hipStream_t)stream, "gemm");
}

extern "C" int clarus_hip_conv3x3(const ClarusConvArgs* a, void* stream) {
  clear_error();
  CLARUS_REQUIRE(a != nullptr, "conv3x3: null args");
  CLARUS_REQUIRE(a->x && a->wt && a->out, "conv3x3: null operand");
  CLARUS_REQUIRE(a->batch > 0 && a->h > 0 && a->w > 0 && a->cin > 0 && a->cout > 0, "conv3x3: empty problem");
  CLARUS_REQUIRE(dt_ok(a->x_dtype) && dt_ok(a->w_dtype) && dt_ok(a->o_dtype), "conv3x3: bad dtype code");
  CLARUS_REQUIRE(a->cin % 8 == 0, "conv3x3: cin=%lld must be a multiple of 8", (long long)a->cin);
  CLARUS_REQUIRE(a->act == ACT_NONE || a->act == ACT_LRELU, "conv3x3: act must be none or lrelu");
  CLARUS_REQUIRE(a->c_mode == CLARUS_C_ROWS || a->c_mode == CLARUS_C_NCHW, "conv3x3: bad c_mode");
  const int ex = esize(a->x_dtype);
  CLARUS_REQUIRE(aligned(a->x, 16) && (a->ldx * ex) % 16 == 0 && a->ldx >= a->cin,
                 "conv3x3: x must be 16-byte aligned with a 16-byte pixel stride");
  CLARUS_REQUIRE(aligned(a->wt, 16), "conv3x3: weights must be 16-byte aligned");
  if (a->res) CLARUS_REQUIRE(dt_ok(a->r_dtype), "conv3x3: bad residual dtype");

  GemmP p{};
  const int64_t H = a->h << (a->up2 ? 1 : 0), W = a->w << (a->up2 ? 1 : 0);
  p.a = a->x; p.wt = a->wt; p.c = a->out;
  p.bias = a->bias; p.scale = nullptr; p.res = a->res;
  p.m = a->batch * H * W; p.n = a->cout; p.k = 9 * a->cin;
  p.lda = a->ldx; p.ldc = a->ldo; p.ldr = a->ldr;
  p.c_dt = a->o_dtype; p.r_dt = a->r_dtype;
  p.h = (int)a->h; p.w = (int)a->w; p.cin = (int)a->cin; p.up2 = a->up2 ? 1 : 0;
  p.pro = PRO_NONE; p.c_mode = a->c_mode; p.act = a->act;
  p.has_res = a->res != nullptr;
  p.out_scale = a->out_scale; p.slope = a->slope; p.ln_eps = 0.f;
  const int eo = esize(a->o_dtype);
  if (a->c_mode == CLARUS_C_ROWS) {
    CLARUS_REQUIRE(a->ldo >= a->cout && (!a->res || a->ldr >= a->cout), "conv3x3: pixel strides smaller than cout");
    p.vec_out = vec_level(a->out, eo, a->ldo, 0);
    p.vec_res = a->res ? vec_level(a->res, esize(a->r_dtype), a->ldr, 0) : 0;
  } else {
    p.vec_out = 0;
    p.vec_res = 0;
  }
  const int opm = operand_mode(a->x_dtype, a->w_dtype, false);
  // output tiles with an LDS halo and resident weights (tile 0 = auto, 12 = force); the
  // implicit GEMM otherwise (tiles 1..7)
  const bool halo_ok = opm == OPM_BF16 && (a->c_mode == CLARUS_C_ROWS || (a->c_mode == CLARUS_C_NCHW && !a->up2)) &&
                       a->cin % 32 == 0 && a->batch * H * W < ((int64_t)1 << 31);
  CLARUS_REQUIRE(a->tile != 12 || halo_ok, "conv3x3: the halo-tile kernel does not take this problem");
  if (halo_ok && (a->tile == 0 || a->tile == 12)) {
    note_kernel("conv_halo_kernel up2=%d", p.up2);
    if (launch_conv_halo(p, (hipStream_t)stream)) return check_launch("conv3x3");
    CLARUS_REQUIRE(a->tile == 0, "conv3x3: the halo-tile kernel's weights do not fit in LDS");
  }
  const int tile = a->tile > 0 ? a->tile - 1 : auto_tile(p.m, p.n, p.k, 1, false, opm, 0);
  note_kernel("gemm_kernel tile=%d am=conv3 opm=%d", tile + 1, opm);
  return launch(p, AM_CONV3, false, opm, a->x_dtype, tile, 1, (hipStream_t)stream, "conv3x3");
}

// ------------------------------------------------------------------- intro 3 -> C conv
// One thread per (pixel, 8 output channels), lanes channel-group-minor so a wave stores whole
// pixel rows: 27 input loads (shared through L1 by the threads of a pixel), 27 x 8 fp32 FMAs
// with the taps read from LDS as 16-byte vectors, one 16-byte bf16 store (two for fp32).
// Persistent grid; all index math in 32 bits (the host checks the sizes).
template <int ODT>
__global__ void __launch_bounds__(256) intro_kernel(const float* __restrict__ inp, const float* __restrict__ wt,
                                                    const float* __restrict__ bias, void* out, int m, int h,
                                                    int w, int cout) {
  extern __shared__ __attribute__((aligned(16))) float wsh[];  // [27][cout] taps, then [cout] bias
  for (int i = threadIdx.x; i < 28 * cout; i += 256) wsh[i] = i < 27 * cout ? wt[i] : bias[i - 27 * cout];
  __syncthreads();
  const int groups = cout >> 3;
  const int total = m * groups;
  const int hw = h * w;
  for (int t = blockIdx.x * 256 + threadIdx.x; t < total; t += gridDim.x * 256) {
    const int q = t / groups;
    const int c0 = (t - q * groups) * 8;
    const int img = q / hw;
    const int rr = q - img * hw;
    const int y = rr / w, x = rr - (rr / w) * w;
    const float* plane = inp + (int64_t)img * 3 * hw;
    f32x4 a0 = *reinterpret_cast<const f32x4*>(wsh + 27 * cout + c0);
    f32x4 a1 = *reinterpret_cast<const f32x4*>(wsh + 27 * cout + c0 + 4);
#pragma unroll
    for (int ky = 0; ky < 3; ++ky) {
      const int yy = y + ky - 1;
      if (yy < 0 || yy >= h) continue;
#pragma unroll
      for (int kx = 0; kx < 3; ++kx) {
        const int xx = x + kx - 1;
        if (xx < 0 || xx >= w) continue;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
          const float v = plane[c * hw + yy * w + xx];
          const float* wr = wsh + ((ky * 3 + kx) * 3 + c) * cout + c0;
          const f32x4 w0 = *reinterpret_cast<const f32x4*>(wr);
          const f32x4 w1 = *reinterpret_cast<const f32x4*>(wr + 4);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            a0[i] = fmaf(v, w0[i], a0[i]);
            a1[i] = fmaf(v, w1[i], a1[i]);
          }
        }
      }
    }
    const int64_t oo = (int64_t)q * cout + c0;
    if constexpr (ODT == DT_BF16) {
      u32x4 r;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        r[i] = (unsigned)f32_to_bf16_bits(a0[2 * i]) | ((unsigned)f32_to_bf16_bits(a0[2 * i + 1]) << 16);
        r[2 + i] = (unsigned)f32_to_bf16_bits(a1[2 * i]) | ((unsigned)f32_to_bf16_bits(a1[2 * i + 1]) << 16);
      }
      *reinterpret_cast<u32x4*>((unsigned short*)out + oo) = r;
    } else {
      *reinterpret_cast<f32x4*>((float*)out + oo) = a0;
      *reinterpret_cast<f32x4*>((float*)out + oo + 4) = a1;
    }
  }
}

// MFMA form for cout % 64 == 0: the 3 x 3 x 3 taps are K = 27 (padded to 28) of an fp32
// 16x16x4 MFMA product D[channel][pixel] = W^T[channel][k] . A[k][pixel], fp32 products and
// fp32 accumulation like the FMA kernel above (only the summation order differs). A wave takes
// 16 consecutive pixels x 64 channels per step: lane l loads the 7 input values k = 4 s + l / 16
// (s < 7) of pixel l % 16 straight from the NCHW planes (16 consecutive floats per tap row and
// channel), holds its 28 W^T operands for the whole kernel, and issues 7 x 4 MFMAs. W^T rows are
// permuted so lane group g = l / 16 ends with channels 8 g .. 8 g + 7 and 32 + 8 g .. 32 + 8 g + 7
// of its pixel: each 16-byte store of the four groups covers 64 contiguous bytes of a pixel row.
template <int ODT>
__global__ void __launch_bounds__(256) intro_mfma_kernel(const float* __restrict__ inp, const float* __restrict__ wt,
                                                         const float* __restrict__ bias, void* out, int m, int h,
                                                         int w, int cout) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int hw = h * w;
  const int ncg = cout >> 6;                  // 64-channel groups
  const int nblk = (m + 15) >> 4;             // 16-pixel blocks
  const int units = nblk * ncg;
  int kc[7], koff[7], kdy[7], kdx[7];         // this lane's k of each step: channel plane, tap offsets
#pragma unroll
  for (int s = 0; s < 7; ++s) {
    const int k = 4 * s + g;
    const int kk = k < 27 ? k : 0;
    const int tap = kk / 3, c = kk - 3 * tap;
    kc[s] = k < 27 ? c : -1;
    kdy[s] = tap / 3 - 1;
    kdx[s] = tap - 3 * (tap / 3) - 1;
    koff[s] = c * hw + kdy[s] * w + kdx[s];
  }
  int cg_cur = -1;
  float wv[4][7], bv[16];
  for (int u = blockIdx.x * 4 + wave; u < units; u += gridDim.x * 4) {
    const int cg = u / nblk, blk = u - cg * nblk;
    if (cg != cg_cur) {  // W^T operands and bias of the channel group (once per wave when ncg == 1)
      cg_cur = cg;
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        const int ch = cg * 64 + (cb >> 1) * 32 + 8 * (j >> 2) + 4 * (cb & 1) + (j & 3);
#pragma unroll
        for (int s = 0; s < 7; ++s) wv[cb][s] = kc[s] >= 0 ? wt[(4 * s + g) * cout + ch] : 0.f;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) bv[i] = bias[cg * 64 + (i >> 3) * 32 + 8 * g + (i & 7)];
    }
    const int q = blk * 16 + j;
    const bool qok = q < m;
    const int qq = qok ? q : m - 1;
    const int img = qq / hw;
    const int rr = qq - img * hw;
    const int y = rr / w, x = rr - (rr / w) * w;
    const float* plane = inp + (int64_t)img * 3 * hw + rr;
    float a[7];
#pragma unroll
    for (int s = 0; s < 7; ++s) {
      const int yy = y + kdy[s], xx = x + kdx[s];
      const bool ok = kc[s] >= 0 && yy >= 0 && yy < h && xx >= 0 && xx < w;
      a[s] = ok ? plane[koff[s]] : 0.f;
    }
    f32x4 acc[4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      acc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 7; ++s) acc[cb] = mfma_f32(wv[cb][s], a[s], acc[cb]);
    }
    if (!qok) continue;
    float v[16];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int i = 0; i < 4; ++i) v[(cb >> 1) * 8 + (cb & 1) * 4 + i] = acc[cb][i] + bv[(cb >> 1) * 8 + (cb & 1) * 4 + i];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int64_t oo = (int64_t)q * cout + cg * 64 + hf * 32 + 8 * g;
      if constexpr (ODT == DT_BF16) {
        u32x4 r;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          r[i] = (unsigned)f32_to_bf16_bits(v[hf * 8 + 2 * i]) | ((unsigned)f32_to_bf16_bits(v[hf * 8 + 2 * i + 1]) << 16);
        *reinterpret_cast<u32x4*>((unsigned short*)out + oo) = r;
      } else {
        *reinterpret_cast<f32x4*>((float*)out + oo) = f32x4{v[hf * 8], v[hf * 8 + 1], v[hf * 8 + 2], v[hf * 8 + 3]};
        *reinterpret_cast<f32x4*>((float*)out + oo + 4) =
            f32x4{v[hf * 8 + 4], v[hf * 8 + 5], v[hf * 8 + 6], v[hf * 8 + 7]};
      }
    }
  }
}

extern "C" int clarus_hip_intro3x3(const float* inp, const float* wt, const float* bias, void* out,
                                   int32_t out_dtype, int64_t batch, int64_t h, int64_t w, int64_t cout,
                                   void* stream) {
  clear_error();
  CLARUS_REQUIRE(inp && wt && bias && out, "intro3x3: null operand");
  CLARUS_REQUIRE(batch > 0 && h > 0 && w > 0 && cout > 0, "intro3x3: empty problem");
  CLARUS_REQUIRE(dt_ok(out_dtype), "intro3x3: bad dtype");
  CLARUS_REQUIRE(cout % 8 == 0 && cout <= 512, "intro3x3: cout must be a multiple of 8, at most 512");
  CLARUS_REQUIRE(batch * h * w * (cout / 8) < ((int64_t)1 << 31), "intro3x3: problem too large for 32-bit indexing");
  CLARUS_REQUIRE(aligned(out, 16) && aligned(wt, 16) && aligned(bias, 16), "intro3x3: 16-byte alignment");
  const int64_t m = batch * h * w;
  if (cout % 64 == 0 && batch * h * w * 3 < ((int64_t)1 << 31)) {
    const int64_t units = cdiv(m, 16) * (cout / 64);
    const unsigned blocks = (unsigned)std::min<int64_t>(cdiv(units, 4), 8LL * device_cus());
    if (out_dtype == DT_BF16)
      hipLaunchKernelGGL(intro_mfma_kernel<DT_BF16>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, inp, wt, bias,
                         out, (int)m, (int)h, (int)w, (int)cout);
    else
      hipLaunchKernelGGL(intro_mfma_kernel<DT_F32>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, inp, wt, bias,
                         out, (int)m, (int)h, (int)w, (int)cout);
    return check_launch("intro3x3");
  }
  const int64_t work = m * (cout / 8);
  const size_t lds = (size_t)28 * cout * sizeof(float);
  const unsigned blocks = (unsigned)std::min<int64_t>(cdiv(work, 256), 8LL * device_cus());
  if (out_dtype == DT_BF16)
    hipLaunchKernelGGL(intro_kernel<DT_BF16>, dim3(blocks), dim3(256), lds, (hipStream_t)stream, inp, wt, bias, out,
                       (int)m, (int)h, (int)w, (int)cout);
  else
    hipLaunchKernelGGL(intro_kernel<DT_F32>, dim3(blocks), dim3(256), lds, (hipStream_t)stream, inp, wt, bias, out,
                       (int)m, (int)h, (int)w, (int)cout);
  return check_launch("intro3x3");
}
