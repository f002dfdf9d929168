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
#include <type_traits>

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

// The second GEMM of clarus_hip_gemm_ln_gemm: out2 = gate?((LN rows) . W2 + bias2), K = RL_N.
// Its A operand (the tile's normalised rows) stays in LDS; its W^T fragments stream straight
// from global memory into registers, each wave its own 64 W^T rows, so the loop has no barrier.
// w2p holds them in fragment order: pass P (512 W^T rows), wave w, 16-k step s, block b (32 rows),
// lane l: the 8 values W^T[row(P, 64 w + 32 b + l % 32)][16 s + 8 (l / 32) + e] (one 1 KiB load
// per fragment; a wave's 64-k group is 8 KiB contiguous).
constexpr int L2_ROWS = 512;                     // W^T rows per pass
constexpr int L2_STEPS = RL_N / 16;              // 16-k steps per pass (32)
constexpr int L2_GROUPS = L2_STEPS / 4;          // 64-k groups per pass (8)
constexpr int L2_A = 0;                          // LN rows: 64 rows x 1 KiB, units XOR (row % 16)
constexpr int L2_OUT = RL_P * RL_N * 2;          // a pass's output per wave: 64 pixels x 64 channels bf16
constexpr int L2_OUT_WAVE = RL_P * 64 * 2;       // 8 KiB per wave
static_assert(L2_OUT + RL_WAVES * L2_OUT_WAVE <= RL_RING, "the LN rows and the output staging reuse the ring");

struct Ln2P {
  const void* w2p;     // packed W^T rows (above), bf16
  const float* bias2;  // [n2w] fp32 (W^T row order), or null
  void* out2;          // [m][ld2] bf16
  int64_t ld2;
  int n2w;             // W^T rows: a multiple of 512
  int gate;            // SimpleGate: out2 channel c = (row c) * (row c + n2w / 2)
};

template <bool FUSE>
__global__ void __launch_bounds__(RL_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
gemm_rowln_kernel(const GemmP p, const RowLnP q, const Ln2P r2) {
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
    if constexpr (!FUSE) {
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
    }
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.f;
    if constexpr (FUSE) {
      // ---- second GEMM on the tile's normalised rows, which stay in LDS (a workgroup has one
      // tile: the host launches one workgroup per tile). Every wave is past its staging reads
      // (the last statistics barrier above), so the ring is free for the rows (at L2_A). Its 8
      // waves compute 64 pixels x 64 W^T rows each per 512-row pass, as in the first GEMM, with
      // the W^T fragments of the next 64-k group in flight while one group is multiplied.
      // lane and wave indices laundered here, so the compiler cannot hoist this phase's
      // address arithmetic above the first GEMM (where it would hold registers through its loop)
      int lane_f = lane, wave_f = wave;
      asm volatile("" : "+v"(lane_f), "+v"(wave_f));
      const int l32f = lane_f & 31, hlf = lane_f >> 5;
      const int npass = r2.n2w / L2_ROWS;
      const int total = npass * L2_GROUPS;  // 64-k groups
      const unsigned char* W2 = (const unsigned char*)r2.w2p + ((int64_t)wave_f * L2_STEPS * 2 * 64 + lane_f) * 16;
      bf16x8 wf2[2][4][2];  // [buffer][16-k step][block]
      auto load_group = [&](int buf, int g) __attribute__((always_inline)) {
        // group g = pass g / 8, steps 4 (g % 8) .. + 3
        const unsigned char* src = W2 + ((int64_t)(g / L2_GROUPS) * RL_WAVES * L2_STEPS * 2 + (g % L2_GROUPS) * 8) * 1024;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
          for (int rb = 0; rb < 2; ++rb)
            wf2[buf][ks][rb] = *reinterpret_cast<const bf16x8*>(src + (ks * 2 + rb) * 1024);
      };
      load_group(0, 0);
      // rows into LDS: pixel px, 16-byte unit u = 8 wave + lane % 8 of its 64, stored at u ^ (px % 16)
#pragma unroll
      for (int pb = 0; pb < 2; ++pb)
#pragma unroll
        for (int rd = 0; rd < 4; ++rd) {
          const int px = pb * 32 + rd * 8 + (lane_f >> 3);
          f32x8 o;
#pragma unroll
          for (int i = 0; i < 8; ++i) o.v[i] = (yv[pb][rd][i] - mean[pb][rd]) * rstd[pb][rd];
          const int u = wave_f * 8 + (lane_f & 7);
          *reinterpret_cast<bf16x8*>(lds + L2_A + px * (RL_N * 2) + (u ^ (px & 15)) * 16) = pack_bf16(o);
        }
      barrier_keep_vm();  // every wave's rows are in LDS
      const int64_t q0 = (int64_t)t * RL_P;
      // one 64-k group: its A fragments from LDS, 16 MFMAs
      auto group = [&](const int buf, const int g) __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const int ua = (g % L2_GROUPS) * 8 + 2 * ks + hlf;  // 16-byte unit of the 1 KiB row
          bf16x8 af2[2];
#pragma unroll
          for (int pb = 0; pb < 2; ++pb) {
            const int px = pb * 32 + l32f;
            af2[pb] = *reinterpret_cast<const bf16x8*>(lds + L2_A + px * (RL_N * 2) + (ua ^ (px & 15)) * 16);
          }
#pragma unroll
          for (int pb = 0; pb < 2; ++pb)
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) acc[pb][rb] = mfma32_bf16(wf2[buf][ks][rb], af2[pb], acc[pb][rb]);
        }
      };
      // pass epilogue: + bias2 (SimpleGate), rounded once to bf16, through the wave's LDS staging
      // (64 pixel rows of its 64 channels, 32 with the gate; 16-byte units XOR-swizzled by row) so
      // each store instruction writes 8 whole 128-byte row pieces (16 of 64 bytes with the gate)
      // instead of 64 16-byte pieces from the MFMA layout
      unsigned char* so = lds + L2_OUT + wave_f * L2_OUT_WAVE;
      auto pass_epilogue = [&](const int pass) __attribute__((always_inline)) {
        const bool GATE = r2.gate;
        const int upr = GATE ? 4 : 8;  // 16-byte units per staged row
#pragma unroll
        for (int pb = 0; pb < 2; ++pb) {
          const int px = pb * 32 + l32f;
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) {
            if (GATE && rb == 1) continue;
            const int lc = GATE ? 16 * hlf : rb * 32 + 16 * hlf;  // first channel within the wave's run
            const int c0 = GATE ? pass * (L2_ROWS / 2) + wave_f * 32 + lc : pass * L2_ROWS + wave_f * 64 + lc;
            float v[16];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const f32x4 b1 = r2.bias2 ? *reinterpret_cast<const f32x4*>(r2.bias2 + c0 + 4 * i) : f32x4{0.f, 0.f, 0.f, 0.f};
              if (GATE) {
                const f32x4 b2 = r2.bias2 ? *reinterpret_cast<const f32x4*>(r2.bias2 + r2.n2w / 2 + c0 + 4 * i)
                                          : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int e = 0; e < 4; ++e) v[4 * i + e] = (acc[pb][0][4 * i + e] + b1[e]) * (acc[pb][1][4 * i + e] + b2[e]);
              } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) v[4 * i + e] = acc[pb][rb][4 * i + e] + b1[e];
              }
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              f32x8 o;
#pragma unroll
              for (int i = 0; i < 8; ++i) o.v[i] = v[8 * h + i];
              const int u = lc / 8 + h;
              *reinterpret_cast<bf16x8*>(so + px * upr * 16 + (u ^ (px & (upr - 1))) * 16) = pack_bf16(o);
            }
          }
        }
        // read back in row order (the wave's own staging: its LDS accesses stay in order)
        const int ppi = 64 / upr;  // pixels per store instruction
        const int c_base = GATE ? pass * (L2_ROWS / 2) + wave_f * 32 : pass * L2_ROWS + wave_f * 64;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          if (j * ppi >= RL_P) break;
          const int px = j * ppi + lane_f / upr, u = lane_f % upr;
          const bf16x8 ov = *reinterpret_cast<const bf16x8*>(so + px * upr * 16 + (u ^ (px & (upr - 1))) * 16);
          const int64_t qq = q0 + px;
          if (qq < p.m) *reinterpret_cast<bf16x8*>((unsigned char*)r2.out2 + (qq * r2.ld2 + c_base + u * 8) * 2) = ov;
        }
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
          for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.f;
      };
      // groups in pairs (register buffers 0 / 1 by constant index); total is even (8 per pass).
      // Loads return in order, so vmcnt(8) (the next group's 8 loads outstanding) means group g
      // has landed, whatever epilogue stores are still in flight.
      for (int g = 0; g < total; g += 2) {
        load_group(1, g + 1);
        wait_vmcnt<8>();
        group(0, g);
        if ((g + 1) % L2_GROUPS == 0) pass_epilogue(g / L2_GROUPS);
        if (g + 2 < total) {
          load_group(0, g + 2);
          wait_vmcnt<8>();
        } else {
          wait_vmcnt<0>();
        }
        group(1, g + 1);
        if ((g + 2) % L2_GROUPS == 0) pass_epilogue((g + 1) / L2_GROUPS);
      }
    }
  }
}

}  // namespace

}  // namespace clarus

using namespace clarus;

namespace {

// checks shared by both entry points; fills the first GEMM's parameters
int rowln_params(const ClarusGemmArgs* a, const void* ln_out, float eps, int32_t rms, GemmP& p, const char* what) {
  CLARUS_REQUIRE(a != nullptr && a->a && a->wt && a->c && ln_out, "%s: null operand", what);
  CLARUS_REQUIRE(a->m > 0 && a->k > 0, "%s: empty problem", what);
  CLARUS_REQUIRE(a->n == RL_N, "%s: N=%lld, the row tile covers exactly %d channels", what, (long long)a->n, RL_N);
  CLARUS_REQUIRE(a->a_dtype == DT_BF16 && a->w_dtype == DT_BF16, "%s: bf16 A and W", what);
  CLARUS_REQUIRE(a->c_dtype == DT_BF16 || a->c_dtype == DT_F32, "%s: bad output dtype", what);
  CLARUS_REQUIRE(!a->res || a->r_dtype == DT_BF16 || a->r_dtype == DT_F32, "%s: bad residual dtype", what);
  CLARUS_REQUIRE(a->a_mode == CLARUS_A_ROWS && a->c_mode == CLARUS_C_ROWS && a->batch == 1 && a->pro == PRO_NONE &&
                     !a->gate && a->act == ACT_NONE,
                 "%s: plain rows (no prologue, gate, activation, batch or pixel shuffle)", what);
  CLARUS_REQUIRE(a->k % M32_KC == 0, "%s: K=%lld must be a multiple of %d", what, (long long)a->k, M32_KC);
  CLARUS_REQUIRE(a->lda >= a->k && (a->lda * 2) % 16 == 0 && aligned(a->a, 16) && aligned(a->wt, 16),
                 "%s: 16-byte A / W rows", what);
  const int ec = a->c_dtype == DT_BF16 ? 2 : 4, er = a->r_dtype == DT_BF16 ? 2 : 4;
  CLARUS_REQUIRE(a->ldc >= a->n && (a->ldc * ec) % 16 == 0 && aligned(a->c, 16), "%s: 16-byte output rows", what);
  CLARUS_REQUIRE(!a->res || (a->ldr >= a->n && (a->ldr * er) % 16 == 0 && aligned(a->res, 16)),
                 "%s: 16-byte residual rows", what);
  CLARUS_REQUIRE(aligned(ln_out, 16), "%s: 16-byte normalised rows", what);
  CLARUS_REQUIRE(eps >= 0.f && (rms == 0 || rms == 1), "%s: bad eps / mode", what);
  CLARUS_REQUIRE(cdiv(a->m, RL_P) < ((int64_t)1 << 31), "%s: too many tiles", what);
  p = GemmP{};
  p.a = a->a; p.wt = a->wt; p.c = a->c;
  p.bias = a->bias; p.scale = a->scale; p.res = a->res;
  p.m = a->m; p.n = a->n; p.k = a->k;
  p.lda = a->lda; p.ldc = a->ldc; p.ldr = a->ldr;
  p.c_dt = a->c_dtype; p.r_dt = a->r_dtype;
  p.has_res = a->res != nullptr;
  p.out_scale = a->out_scale;
  p.ptiles = cdiv(a->m, RL_P);
  return CLARUS_OK;
}

template <bool FUSE>
int rowln_launch(const GemmP& p, const RowLnP& q, const Ln2P& r2, void* stream, const char* what) {
  static const int per_cu = [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_rowln_kernel<FUSE>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(&gemm_rowln_kernel<FUSE>),
                                                     RL_THREADS, RL_LDS) != hipSuccess ||
        n < 1)
      n = 1;
    return n;
  }();
  // one tile per workgroup at most (the fused second GEMM reuses the ring, so a workgroup
  // cannot prefetch a next tile); without the fusion, persistent up to the resident count
  const int64_t need = cdiv(p.ptiles, 8) * 8;
  int64_t gx = FUSE ? need : std::min<int64_t>((int64_t)device_cus() * per_cu, need);
  note_kernel("gemm_rowln_kernel fuse=%d", (int)FUSE);
  hipLaunchKernelGGL(gemm_rowln_kernel<FUSE>, dim3((unsigned)gx), dim3(RL_THREADS), RL_LDS, (hipStream_t)stream, p,
                     q, r2);
  return check_launch(what);
}

}  // namespace

extern "C" int clarus_hip_gemm_ln_rows(const ClarusGemmArgs* a, void* ln_out, float eps, int32_t rms, void* stream) {
  clear_error();
  GemmP p;
  if (int rc = rowln_params(a, ln_out, eps, rms, p, "gemm_ln_rows")) return rc;
  return rowln_launch<false>(p, RowLnP{ln_out, eps, rms}, Ln2P{}, stream, "gemm_ln_rows");
}

extern "C" int clarus_hip_gemm_ln_gemm(const ClarusGemmArgs* a, float eps, int32_t rms, const void* w2p,
                                       const float* bias2, void* out2, int64_t n2w, int32_t gate2, void* stream) {
  clear_error();
  GemmP p;
  if (int rc = rowln_params(a, w2p, eps, rms, p, "gemm_ln_gemm")) return rc;
  CLARUS_REQUIRE(out2 != nullptr && aligned(out2, 16) && aligned(w2p, 16), "gemm_ln_gemm: 16-byte packed W2 / out2");
  CLARUS_REQUIRE(n2w > 0 && n2w % L2_ROWS == 0 && n2w <= (1 << 20), "gemm_ln_gemm: n2w=%lld must be a multiple of %d",
                 (long long)n2w, L2_ROWS);
  CLARUS_REQUIRE(gate2 == 0 || gate2 == 1, "gemm_ln_gemm: gate2 is 0 or 1");
  CLARUS_REQUIRE(bias2 == nullptr || aligned(bias2, 16), "gemm_ln_gemm: 16-byte bias2");
  CLARUS_REQUIRE(cdiv(a->m, RL_P) * 8 < ((int64_t)1 << 31), "gemm_ln_gemm: too many tiles");
  Ln2P r2{w2p, bias2, out2, gate2 ? n2w / 2 : n2w, (int)n2w, gate2};
  return rowln_launch<true>(p, RowLnP{nullptr, eps, rms}, r2, stream, "gemm_ln_gemm");
}
