// GEMM whose epilogue also writes the LayerNorm / RMS-normalised rows of its output:
// clarus_hip_gemm_ln_rows (gfx950).
//
// In NAFNet every level-3 c -> c GEMM with the fp32 residual stream (conv3: y = x + beta .
// conv3(..), conv5: z = y + gamma . conv5(..), N = 512) is followed by a GEMM whose prologue is
// the LayerNorm of that output (conv4, the next block's conv1). The reference normalises those
// rows in a separate pass into the compute dtype (kernels/spatial.py:312 ln_rows, called at
// ops/triton_cuda.py:104); here the producing GEMM computes them in its epilogue, from the fp32
// values it has just stored, so the pass (a re-read of the fp32 rows and a launch) disappears.
//
// The tile is a whole output row: 64 pixels x 512 W^T rows. Its 8 waves split the rows (wave w
// owns output channels 64 w .. 64 w + 63) and compute 64 pixels x 64 channels each on 32x32x16
// bf16 MFMAs (2 x 2 blocks), with the operand staging of gemm_mfma32_kernel: 64-k chunks of A
// (64 rows, 8 KiB) and W^T (512 rows, 64 KiB) travel global -> LDS by direct 16-byte copies
// into a 2-stage ring (144 KiB, one workgroup per CU), rows XOR-swizzled, W^T rows permuted so a
// lane accumulates 16 consecutive channels of one pixel.
// Epilogue per tile, per 32-pixel block of a wave: (acc + bias) * scale in the MFMA layout ->
// fp32 LDS rows -> row layout (8 lanes per pixel, 8 channels each) -> + residual -> store y
// (statistics and normalised rows come from the stored values, i.e. after a bf16 output's
// rounding).
// The wave keeps its 64 values per lane; per-pixel sums over the 8 lanes (shuffles) and the 8
// waves (LDS) give the mean, a second exchange the variance (two-pass, as the reference), then
// (y - mean) * rsqrt(var + eps) is rounded to bf16 and stored as the next GEMM's A rows.
#include <algorithm>

#include "capi.hpp"
#include "gemm_mfma32.hpp"

namespace clarus {

namespace {

constexpr int RL_P = 64;                            // pixels per tile
constexpr int RL_N = 512;                           // output channels (W^T rows) per tile
constexpr int RL_WAVES = RL_N / 64;                 // 8
constexpr int RL_THREADS = 64 * RL_WAVES;           // 512
constexpr int RL_ABYTES = RL_P * M32_ROWB;          // 8 KiB
constexpr int RL_WBYTES = RL_N * M32_ROWB;          // 64 KiB
constexpr int RL_STAGE = RL_ABYTES + RL_WBYTES;     // 72 KiB
constexpr int RL_COPIES = RL_STAGE / 1024 / RL_WAVES;  // 9 copies of 1 KiB per wave per stage
constexpr int RL_RING = 2 * RL_STAGE;               // 144 KiB
constexpr int RL_TABLES = 2 * RL_N * 4;             // bias, scale * out_scale
constexpr int RL_RED = 2 * RL_WAVES * RL_P * 4;     // per-wave pixel partials: sums, squares
constexpr int RL_LDS = RL_RING + RL_TABLES + RL_RED;  // 152 KiB
static_assert(RL_ABYTES / 1024 == RL_WAVES, "copy j = 0 of every wave is the A KiB, j >= 1 are W^T");
static_assert(RL_WAVES * EPI32_STAGE_BYTES <= RL_STAGE, "epilogue staging fits one ring stage");
static_assert(RL_LDS <= 160 * 1024, "LDS");

struct RowLnP {
  void* ln_out;  // [m][RL_N] bf16
  float eps;
  int rms;
};

__global__ void __launch_bounds__(RL_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
gemm_rowln_kernel(const GemmP p, const RowLnP q) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  unsigned char* ring = lds;
  float* tb = reinterpret_cast<float*>(lds + RL_RING);                 // [0, 512) bias, [512, 1024) scale
  float* red = reinterpret_cast<float*>(lds + RL_RING + RL_TABLES);    // [2][8 waves][64 pixels]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hl = lane >> 5;
  const int64_t K = p.k;
  const int nch = (int)(K / M32_KC);
  const int T = (int)p.ptiles;
  const unsigned char* A = (const unsigned char*)p.a;
  const unsigned char* Wt = (const unsigned char*)p.wt;

  // tiles dealt out XCD-aware: a contiguous tile range per XCD
  const int xcd = blockIdx.x & 7;
  const int per = gridDim.x >> 3;
  const int span = (T + 7) >> 3;
  const int t0 = xcd * span + (blockIdx.x >> 3);
  const int t_end = (xcd + 1) * span < T ? (xcd + 1) * span : T;
  const int ntiles = t0 < t_end ? (t_end - t0 + per - 1) / per : 0;
  const int nsteps = ntiles * nch;
  if (nsteps == 0) return;  // before any LDS or memory traffic

  // copies of one chunk: wave w moves the KiBs w + 8 j (KiB 0-7: A rows 8 w .. 8 w + 7, KiB
  // 8 + i: W^T rows 8 i .. 8 i + 7); lane l fills row l / 8 of its KiB, slot l % 8, with source
  // unit m32_swz(row, slot)
  int is_tile = 0, is_chunk = 0, is_stage = 0;
  const unsigned char* src_base[RL_COPIES];
  auto set_issue_tile = [&]() __attribute__((always_inline)) {
    const int t = t0 + is_tile * per;
#pragma unroll
    for (int j = 0; j < RL_COPIES; ++j) {
      if (j == 0) {
        const int row = wave * 8 + (lane >> 3);
        int64_t r = (int64_t)t * RL_P + row;
        if (r > p.m - 1) r = p.m - 1;  // rows past M: any valid row, not stored
        src_base[j] = A + (r * p.lda + m32_swz(row, lane & 7) * 8) * 2;
      } else {
        // W^T row `row` = wave-row wr, block rb, block row rr = 8 g + 4 h + i holds channel
        // 16 h + 4 g + i of its 32-channel run
        const int row = (wave + 8 * j - 8) * 8 + (lane >> 3);
        const int wr = row >> 6, rb = (row >> 5) & 1, rr = row & 31;
        const int cw = 16 * ((rr >> 2) & 1) + 4 * (rr >> 3) + (rr & 3);
        int64_t c = wr * 64 + rb * 32 + cw;
        if (c > p.n - 1) c = p.n - 1;
        src_base[j] = Wt + (c * K + m32_swz(row, lane & 7) * 8) * 2;
      }
    }
  };
  auto issue = [&]() __attribute__((always_inline)) {
    const int kb = is_chunk * (M32_KC * 2);
    unsigned char* st = ring + is_stage * RL_STAGE;
#pragma unroll
    for (int j = 0; j < RL_COPIES; ++j)
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src_base[j] + kb),
                                       (__attribute__((address_space(3))) void*)(st + (wave + RL_WAVES * j) * 1024), 16,
                                       0, 0);
    is_stage ^= 1;
    if (++is_chunk == nch) {
      is_chunk = 0;
      ++is_tile;
      if (is_tile < ntiles) set_issue_tile();
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.f;

  bf16x8 wf[2][2], af[2][2];
  auto load_frags = [&](int buf, int stage, int ks) __attribute__((always_inline)) {
    const unsigned char* st = ring + stage * RL_STAGE;
    const int u = 2 * ks + hl;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int r = wave * 64 + rb * 32 + l32;
      wf[buf][rb] = *reinterpret_cast<const bf16x8*>(st + RL_ABYTES + r * M32_ROWB + m32_swz(r, u) * 16);
    }
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
      const int r = pb * 32 + l32;
      af[buf][pb] = *reinterpret_cast<const bf16x8*>(st + r * M32_ROWB + m32_swz(r, u) * 16);
    }
  };
  auto products = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) acc[pb][rb] = mfma32_bf16(wf[buf][rb], af[buf][pb], acc[pb][rb]);
  };

  set_issue_tile();
  issue();
  // tables: bias and scale * out_scale of all 512 channels (loads overlap the first copies)
  float tv[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i = tid + j * RL_THREADS;
    const int c = i & (RL_N - 1);
    float x = 0.f;
    if (c < p.n) x = i < RL_N ? (p.bias ? p.bias[c] : 0.f) : (p.scale ? p.scale[c] : 1.f) * p.out_scale;
    tv[j] = x;
  }
  wait_vmcnt<0>();
  barrier_keep_vm();
  if (1 < nsteps) issue();
#pragma unroll
  for (int j = 0; j < 2; ++j) tb[tid + j * RL_THREADS] = tv[j];
  load_frags(0, 0, 0);
  int s = 0, c_stage = 0;

  const int er = p.r_dt == DT_BF16 ? 2 : 4;
  const int ec = p.c_dt == DT_BF16 ? 2 : 4;
  const float invn = 1.0f / (float)p.n;

  for (int tl = 0; tl < ntiles; ++tl) {
    int last_stage = 0;
    bool deferred = false;
    for (int kc = 0; kc < nch; ++kc, ++s) {
#pragma unroll
      for (int ks = 0; ks < M32_KC / 16 - 1; ++ks) {
        load_frags((ks + 1) & 1, c_stage, ks + 1);
        products(ks & 1);
      }
      const int n_stage = c_stage ^ 1;
      if (s + 1 < nsteps) {
        wait_vmcnt<0>();
        barrier_keep_vm();
        if (s + 2 < nsteps) {
          if (kc == nch - 1) deferred = true;
          else issue();
        }
        load_frags(0, n_stage, 0);
      } else {
        barrier_keep_vm();
      }
      last_stage = c_stage;
      products(1);
      c_stage = n_stage;
    }

    // ---- epilogue: y = (acc + bias) * scale (+ residual), kept as yv[pb][rd][8] in the row
    // layout (pixel pb * 32 + rd * 8 + lane / 8, channels 64 wave + 8 (lane % 8) + i)
    const int t = t0 + tl * per;
    float* stg = reinterpret_cast<float*>(ring + last_stage * RL_STAGE + wave * EPI32_STAGE_BYTES);
    float yv[2][4][8];
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
      // the block's residual loads first (one memory round trip, overlapping the staging below),
      // into the registers that then take the row values
#pragma unroll
      for (int rd = 0; rd < 4; ++rd) {
        int64_t qq = (int64_t)t * RL_P + pb * 32 + rd * 8 + (lane >> 3);
        if (qq > p.m - 1) qq = p.m - 1;  // rows past M: any valid row, not stored
        f32x8 rv = zero8();
        if (p.has_res) {
          const unsigned char* rp = (const unsigned char*)p.res + (qq * p.ldr + wave * 64 + (lane & 7) * 8) * er;
          rv = p.r_dt == DT_BF16 ? load8<DT_BF16>(rp) : load8<DT_F32>(rp);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) yv[pb][rd][i] = rv.v[i];
      }
#pragma unroll
      for (int ro = 0; ro < 2; ++ro) {
        const int cw = ro * 32 + 16 * hl;  // first channel of this lane's run within the wave
        const int c0 = wave * 64 + cw;
        float v[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x4 b = *reinterpret_cast<const f32x4*>(tb + c0 + 4 * i);
          const f32x4 sc = *reinterpret_cast<const f32x4*>(tb + RL_N + c0 + 4 * i);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[4 * i + e] = (acc[pb][ro][4 * i + e] + b[e]) * sc[e];
        }
        float* rowp = stg + l32 * 64;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *reinterpret_cast<f32x4*>(rowp + 4 * epi32_unit<64>(l32, cw / 4 + i)) =
              f32x4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int rd = 0; rd < 4; ++rd) {
        const int r = rd * 8 + (lane >> 3);
        const int cg = (lane & 7) * 8;
        const float* rowp = stg + r * 64;
        const f32x4 a0 = *reinterpret_cast<const f32x4*>(rowp + 4 * epi32_unit<64>(r, cg / 4));
        const f32x4 a1 = *reinterpret_cast<const f32x4*>(rowp + 4 * epi32_unit<64>(r, cg / 4 + 1));
        float v[8] = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
        const int64_t qq = (int64_t)t * RL_P + pb * 32 + r;
        const int64_t ch = wave * 64 + cg;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] += yv[pb][rd][i];  // the residual (0 without one)
        if (qq < p.m) {
          unsigned char* op = (unsigned char*)p.c + (qq * p.ldc + ch) * ec;
          if (p.c_dt == DT_BF16) {  // the rows are normalised from the stored (rounded) values
            f32x8 o;
#pragma unroll
            for (int i = 0; i < 8; ++i) o.v[i] = v[i];
            const bf16x8 ob = pack_bf16(o);
            *reinterpret_cast<bf16x8*>(op) = ob;
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = (float)ob[i];
          } else {
            *reinterpret_cast<f32x4*>(op) = f32x4{v[0], v[1], v[2], v[3]};
            *reinterpret_cast<f32x4*>(op + 16) = f32x4{v[4], v[5], v[6], v[7]};
          }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) yv[pb][rd][i] = v[i];
      }
      asm volatile("" ::: "memory");  // the next block's staging writes follow these reads (same wave)
    }

    // ---- row statistics over the 512 channels: 8 lanes of a pixel (shuffles), 8 waves (LDS);
    // two passes like the reference (mean, then the mean of squared deviations)
    float mean[2][4], rstd[2][4];
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      if (pass == 1 || !q.rms) {
#pragma unroll
        for (int pb = 0; pb < 2; ++pb)
#pragma unroll
          for (int rd = 0; rd < 4; ++rd) {
            float acc1 = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const float d = pass == 0 ? yv[pb][rd][i] : yv[pb][rd][i] - mean[pb][rd];
              acc1 += pass == 0 ? d : d * d;
            }
            acc1 += __shfl_xor(acc1, 1, 64);
            acc1 += __shfl_xor(acc1, 2, 64);
            acc1 += __shfl_xor(acc1, 4, 64);
            if ((lane & 7) == 0) red[(pass * RL_WAVES + wave) * RL_P + pb * 32 + rd * 8 + (lane >> 3)] = acc1;
          }
        barrier_keep_vm();
        if (pass == 0 && deferred) {  // every wave is past its staging rows: refill the stage
          issue();
          deferred = false;
        }
#pragma unroll
        for (int pb = 0; pb < 2; ++pb)
#pragma unroll
          for (int rd = 0; rd < 4; ++rd) {
            const int px = pb * 32 + rd * 8 + (lane >> 3);
            float tot = 0.f;
#pragma unroll
            for (int w = 0; w < RL_WAVES; ++w) tot += red[(pass * RL_WAVES + w) * RL_P + px];
            if (pass == 0) mean[pb][rd] = tot * invn;
            else rstd[pb][rd] = rsqrtf(tot * invn + q.eps);
          }
      } else {
#pragma unroll
        for (int pb = 0; pb < 2; ++pb)
#pragma unroll
          for (int rd = 0; rd < 4; ++rd) mean[pb][rd] = 0.f;  // RMS: no centring
      }
    }
    if (deferred) {  // RMS rows: the first exchange was skipped
      barrier_keep_vm();
      issue();
    }

    // ---- normalised rows, rounded once to bf16
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int rd = 0; rd < 4; ++rd) {
        const int64_t qq = (int64_t)t * RL_P + pb * 32 + rd * 8 + (lane >> 3);
        if (qq >= p.m) continue;
        f32x8 o;
#pragma unroll
        for (int i = 0; i < 8; ++i) o.v[i] = (yv[pb][rd][i] - mean[pb][rd]) * rstd[pb][rd];
        *reinterpret_cast<bf16x8*>((unsigned short*)q.ln_out + qq * RL_N + wave * 64 + (lane & 7) * 8) = pack_bf16(o);
      }
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.f;
  }
}

}  // namespace

}  // namespace clarus

using namespace clarus;

extern "C" int clarus_hip_gemm_ln_rows(const ClarusGemmArgs* a, void* ln_out, float eps, int32_t rms, void* stream) {
  clear_error();
  CLARUS_REQUIRE(a != nullptr && a->a && a->wt && a->c && ln_out, "gemm_ln_rows: null operand");
  CLARUS_REQUIRE(a->m > 0 && a->k > 0, "gemm_ln_rows: empty problem");
  CLARUS_REQUIRE(a->n == RL_N, "gemm_ln_rows: N=%lld, the row tile covers exactly %d channels", (long long)a->n, RL_N);
  CLARUS_REQUIRE(a->a_dtype == DT_BF16 && a->w_dtype == DT_BF16, "gemm_ln_rows: bf16 A and W");
  CLARUS_REQUIRE(a->c_dtype == DT_BF16 || a->c_dtype == DT_F32, "gemm_ln_rows: bad output dtype");
  CLARUS_REQUIRE(!a->res || a->r_dtype == DT_BF16 || a->r_dtype == DT_F32, "gemm_ln_rows: bad residual dtype");
  CLARUS_REQUIRE(a->a_mode == CLARUS_A_ROWS && a->c_mode == CLARUS_C_ROWS && a->batch == 1 && a->pro == PRO_NONE &&
                     !a->gate && a->act == ACT_NONE,
                 "gemm_ln_rows: plain rows (no prologue, gate, activation, batch or pixel shuffle)");
  CLARUS_REQUIRE(a->k % M32_KC == 0, "gemm_ln_rows: K=%lld must be a multiple of %d", (long long)a->k, M32_KC);
  CLARUS_REQUIRE(a->lda >= a->k && (a->lda * 2) % 16 == 0 && aligned(a->a, 16) && aligned(a->wt, 16),
                 "gemm_ln_rows: 16-byte A / W rows");
  const int ec = a->c_dtype == DT_BF16 ? 2 : 4, er = a->r_dtype == DT_BF16 ? 2 : 4;
  CLARUS_REQUIRE(a->ldc >= a->n && (a->ldc * ec) % 16 == 0 && aligned(a->c, 16), "gemm_ln_rows: 16-byte output rows");
  CLARUS_REQUIRE(!a->res || (a->ldr >= a->n && (a->ldr * er) % 16 == 0 && aligned(a->res, 16)),
                 "gemm_ln_rows: 16-byte residual rows");
  CLARUS_REQUIRE(aligned(ln_out, 16), "gemm_ln_rows: 16-byte normalised rows");
  CLARUS_REQUIRE(eps >= 0.f && (rms == 0 || rms == 1), "gemm_ln_rows: bad eps / mode");
  CLARUS_REQUIRE(cdiv(a->m, RL_P) < ((int64_t)1 << 31), "gemm_ln_rows: too many tiles");
  GemmP p{};
  p.a = a->a; p.wt = a->wt; p.c = a->c;
  p.bias = a->bias; p.scale = a->scale; p.res = a->res;
  p.m = a->m; p.n = a->n; p.k = a->k;
  p.lda = a->lda; p.ldc = a->ldc; p.ldr = a->ldr;
  p.c_dt = a->c_dtype; p.r_dt = a->r_dtype;
  p.has_res = a->res != nullptr;
  p.out_scale = a->out_scale;
  p.ptiles = cdiv(a->m, RL_P);
  RowLnP q{ln_out, eps, rms};
  static const int per_cu = [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_rowln_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(&gemm_rowln_kernel),
                                                     RL_THREADS, RL_LDS) != hipSuccess ||
        n < 1)
      n = 1;
    return n;
  }();
  int64_t gx = 256LL * per_cu;
  const int64_t need = cdiv(p.ptiles, 8) * 8;
  if (gx > need) gx = need;
  hipLaunchKernelGGL(gemm_rowln_kernel, dim3((unsigned)gx), dim3(RL_THREADS), RL_LDS, (hipStream_t)stream, p, q);
  return check_launch("gemm_ln_rows");
}
