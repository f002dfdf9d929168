// The fused residual GEMM -> LayerNorm -> GEMM pair with both weights streamed from L2 into
// registers: clarus_hip_gemm_ln_gemm_w1p (gfx950), for K = N = 512 (NAFNet level 3: conv3 ->
// conv4, conv5 -> the next block's conv1).
//
// One workgroup of 8 waves per 64-pixel tile, one tile per workgroup, 160 KiB of LDS:
//   [0, 24 KiB)      A ring: 3 stages of 64 rows x 64 k (bf16, 128-byte rows, units swizzled)
//   [24, 152 KiB)    the tile's fp32 residual [64][512] (2 KiB rows, units XOR (row % 8)),
//                    copied by direct global -> LDS loads during the K loop; in the second GEMM
//                    the LN rows [64][512] bf16 (1 KiB rows, units XOR (row % 16)) and each wave's
//                    output staging (8 KiB) take its place
//   [152, 156 KiB)   bias and scale * out_scale of the 512 channels
//   [156, 160 KiB)   per-wave partial sums of the row statistics
// Phase 1 (y = (A W1 + bias) scale + residual): wave w computes 64 pixels x 64 channels (2 x 2
// blocks of 32x32x16 MFMAs). A chunks (64 k) are shared by all waves through the ring; W1 reaches
// each wave's registers straight from L2, packed in fragment order (1 KiB per load, 8 per 64-k
// group), one group ahead. Per chunk the LDS carries 8 KiB of copies and 64 KiB of A fragment
// reads; staging W1 through LDS as well (gemm_rowln_kernel) put 200 KiB per chunk on it.
// Epilogue in the MFMA layout: a lane holds 16 consecutive channels of one pixel per block, adds
// bias, scale and the residual from LDS, stores y, then the two-pass row statistics (lanes, the
// lane pair, the 8 waves through LDS) and the normalised rows into LDS as bf16.
// Phase 2 (out2 = gate?(rows W2 + bias2)): as gemm_rowln_kernel's fused second GEMM.
// replaces kernels/gemm.py:353-400 (fused_gemm) + kernels/spatial.py:312 (ln_rows) + fused_gemm
#include <type_traits>

#include "capi.hpp"
#include "gemm_mfma32.hpp"

namespace clarus {

namespace {

constexpr int PR_P = 64, PR_N = 512, PR_K = 512, PR_WAVES = 8, PR_THREADS = 64 * PR_WAVES;
constexpr int PR_NCH = PR_K / 64;                 // 64-k chunks of the first GEMM
constexpr int PR_STAGE = PR_P * 128;              // 8 KiB
constexpr int PR_STAGES = 3;
constexpr int PR_RES = PR_STAGES * PR_STAGE;      // 24 KiB
constexpr int PR_RES_ROW = PR_N * 4;              // 2 KiB
constexpr int PR_TB = PR_RES + PR_P * PR_RES_ROW; // 152 KiB
constexpr int PR_RED = PR_TB + 2 * PR_N * 4;      // 156 KiB
constexpr int PR_LDS = PR_RED + 2 * PR_WAVES * PR_P * 4;
constexpr int PR_ROWS = PR_RES;                   // second GEMM: LN rows [64][1 KiB]
constexpr int PR_OUT = PR_ROWS + PR_P * PR_N * 2; // second GEMM: 8 KiB output staging per wave
static_assert(PR_LDS == 160 * 1024, "LDS");
static_assert(PR_OUT + PR_WAVES * 8192 <= PR_TB, "second-GEMM regions inside the residual's");

struct PairP {
  const bf16_t* a;      // [m][lda] bf16
  const void* w1p;      // W1^T packed (one 512-row pass)
  const float* bias;    // [512] or null
  const float* scale;   // [512] or null
  const float* res;     // [m][ldr] fp32
  void* c;              // [m][ldc] bf16 / fp32
  const void* w2p;      // W2^T packed
  const float* bias2;   // [n2w] or null
  void* out2;           // [m][ld2] bf16
  int64_t m, lda, ldr, ldc, ld2;
  int c_dt, rms, gate, n2w;
  float eps, out_scale;
  // MUL: A row q times the bf16 map row of its pixel ([n][oh][ow][512], replicate-padded to the
  // h x w image by the offsets pt, pl), the TLC-map prologue of the first GEMM
  const bf16_t* small;
  int h, w, oh, ow, pt, pl;
};

// MUL: each lane multiplies the 16-byte unit it copied of A chunk c by the map values of its row
// (loaded at kernel start), once its own copies have landed and before the barrier that publishes
// the chunk: widened to fp32, multiplied, rounded once to bf16, bit for bit the separate pass's rows.
template <bool CF32, bool GATE, bool MUL>
__global__ void __launch_bounds__(PR_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
pair_kernel(const PairP p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  float* tb = reinterpret_cast<float*>(lds + PR_TB);
  float* red = reinterpret_cast<float*>(lds + PR_RED);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hl = lane >> 5;
  const int64_t t = blockIdx.x;
  const int64_t q0 = t * PR_P;
  if (q0 >= p.m) return;  // before any LDS or memory traffic

  // ---- the packed weights into this XCD's L2 first. Every workgroup reads all of W1 and W2 and
  // they run in step, so from a cold cache each 64-k group would miss at once in all of them, one
  // group ahead of its use. Workgroups go to the XCDs in turn (XCD = block % 8), so the ~28 on an
  // XCD each touch one 128-byte line in 28 of W1 | W2 (at most two per thread; at 720p one). These are
  // the kernel's first memory operations: the first chunk's wait covers them, and the value is
  // only consumed at the end (a dependency the compiler keeps without waiting earlier).
  unsigned int touch[2];
  {
    typedef const __attribute__((address_space(1))) unsigned int* gptr;
    const int xcd = blockIdx.x % 8;
    const int slot = blockIdx.x / 8, nslot = (int)((gridDim.x - xcd + 7) / 8);
    const int lines1 = PR_K * PR_N * 2 / 128, lines = lines1 + PR_K * p.n2w * 2 / 128;
#pragma unroll
    for (int i = 0; i < 2; ++i) {  // two lines per thread at most (the index clamped: no branch)
      int l = (slot + i * nslot) * PR_THREADS + tid;
      l = l < lines ? l : lines - 1;
      const unsigned char* src = l < lines1 ? (const unsigned char*)p.w1p + (int64_t)l * 128
                                            : (const unsigned char*)p.w2p + (int64_t)(l - lines1) * 128;
      touch[i] = *(gptr)(src);
    }
  }
  asm volatile("" ::: "memory");

  // ---- copies. A chunk c (8 KiB): wave w moves rows 8 w .. 8 w + 7, lane l row 8 w + l / 8,
  // slot l % 8 with source unit m32_swz(row, slot). Residual row r (2 KiB, two 1 KiB copies): wave
  // w moves rows 8 w .. 8 w + 7, one per chunk, lane l unit (64 h + l) ^ (r % 8) of half h.
  const int arow = wave * 8 + (lane >> 3);
  int64_t aq = q0 + arow;
  if (aq > p.m - 1) aq = p.m - 1;  // rows past M: any valid row, not stored
  const unsigned char* asrc = (const unsigned char*)(p.a + aq * p.lda) + m32_swz(arow, lane & 7) * 16;
  u32x4 mv[MUL ? PR_NCH : 1];  // map values of this lane's unit in every chunk (chunk 0 waits for all)
  if constexpr (MUL) {
    const int64_t hw = (int64_t)p.h * p.w;
    const int64_t im = aq / hw;
    const int rr = (int)(aq - im * hw);
    const int yq = rr / p.w;
    int sy = yq - p.pt, sx = rr - yq * p.w - p.pl;
    sy = sy < 0 ? 0 : (sy > p.oh - 1 ? p.oh - 1 : sy);
    sx = sx < 0 ? 0 : (sx > p.ow - 1 ? p.ow - 1 : sx);
    const bf16_t* mrow = p.small + ((im * p.oh + sy) * p.ow + sx) * (int64_t)PR_K + m32_swz(arow, lane & 7) * 8;
#pragma unroll
    for (int c = 0; c < PR_NCH; ++c) mv[c] = *reinterpret_cast<const u32x4*>(mrow + c * 64);
    asm volatile("" ::: "memory");
  }
  auto issue_a = [&](int c) __attribute__((always_inline)) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(asrc + c * 128),
                                     (__attribute__((address_space(3))) void*)(lds + (c % PR_STAGES) * PR_STAGE + wave * 1024),
                                     16, 0, 0);
  };
  auto issue_res = [&](int c) __attribute__((always_inline)) {
    const int r = wave * 8 + c;
    int64_t rq = q0 + r;
    if (rq > p.m - 1) rq = p.m - 1;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int u = (64 * h + lane) ^ (r & 7);
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(p.res + rq * p.ldr + u * 4),
                                       (__attribute__((address_space(3))) void*)(lds + PR_RES + r * PR_RES_ROW + h * 1024),
                                       16, 0, 0);
    }
  };
  // W1 group c (k 64 c .. 64 c + 63): 4 16-k steps x 2 blocks of this wave's 64 rows
  const unsigned char* w1 = (const unsigned char*)p.w1p + ((int64_t)wave * (PR_K / 16) * 2 * 64 + lane) * 16;
  bf16x8 wf[2][4][2];
  auto load_w1 = [&](int buf, int c) __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
        wf[buf][ks][rb] = *reinterpret_cast<const bf16x8*>(w1 + ((4 * c + ks) * 2 + rb) * 1024);
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.f;

  // prologue: A chunks 0, 1 and W1 group 0 in flight; the tables go to LDS meanwhile
  issue_a(0);
  issue_a(1);
  asm volatile("" ::: "memory");
  load_w1(0, 0);
  {
    const int c = tid;  // 512 threads: one channel each
    tb[c] = p.bias ? p.bias[c] : 0.f;
    tb[PR_N + c] = (p.scale ? p.scale[c] : 1.f) * p.out_scale;
  }

  // ---- K loop. Issue order per chunk c (after its barrier): W1 group c + 1, A chunk c + 2, the
  // residual rows of chunk c. Loads complete in issue order, so once W1 group c has landed (at most
  // the 3 copies issued after it outstanding: A c + 1 and residual c - 1) so has A chunk c.
  auto chunk = [&](const int buf, const int c) __attribute__((always_inline)) {
    const unsigned char* st = lds + (c % PR_STAGES) * PR_STAGE;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      bf16x8 af[2];
#pragma unroll
      for (int pb = 0; pb < 2; ++pb) {
        const int r = pb * 32 + l32;
        af[pb] = *reinterpret_cast<const bf16x8*>(st + r * 128 + m32_swz(r, 2 * ks + hl) * 16);
      }
#pragma unroll
      for (int pb = 0; pb < 2; ++pb)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) acc[pb][rb] = mfma32_bf16(wf[buf][ks][rb], af[pb], acc[pb][rb]);
    }
  };
#pragma unroll
  for (int c = 0; c < PR_NCH; ++c) {
    // W1 group c and (so) A chunk c have landed: the copies issued after them may stay out
    if (c == 0) wait_vmcnt<0>();  // (the tables' loads, if any, follow W1 group 0)
    else if (c + 1 < PR_NCH) wait_vmcnt<3>();  // after W1 group c: A c + 1, residual c - 1 (2 copies)
    else wait_vmcnt<2>();                      // c = 7: after W1 group 7 only residual 6
    if constexpr (MUL) {  // this lane's unit of chunk c (its copy has landed) times the map
      unsigned char* up = lds + (c % PR_STAGES) * PR_STAGE + wave * 1024 + lane * 16;
      const u32x4 raw = *reinterpret_cast<const u32x4*>(up);
      f32x8 x;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x.v[2 * e] = __uint_as_float(raw[e] << 16) * __uint_as_float(mv[c][e] << 16);
        x.v[2 * e + 1] = __uint_as_float(raw[e] & 0xffff0000u) * __uint_as_float(mv[c][e] & 0xffff0000u);
      }
      *reinterpret_cast<bf16x8*>(up) = pack_bf16(x);
    }
    barrier_keep_vm();                 // every wave's share of A chunk c; chunk c - 1 read by all
    asm volatile("" ::: "memory");
    if (c + 1 < PR_NCH) load_w1((c + 1) & 1, c + 1);
    asm volatile("" ::: "memory");
    if (c + 2 < PR_NCH) issue_a(c + 2);
    issue_res(c);
    asm volatile("" ::: "memory");
    chunk(c & 1, c);
  }

  // ---- epilogue in the MFMA layout: block (pb, rb), lane (l32, hl): pixel pb * 32 + l32,
  // channels 64 wave + 32 rb + 16 hl .. + 15 (element j = channel + j). y stays in registers
  // (yv) and is stored during the second GEMM: stored here, every workgroup's 128 KiB would
  // leave at once and the waves would wait on the write burst before the row statistics.
  wait_vmcnt<0>();
  barrier_keep_vm();  // every residual row in LDS; the tables too
  float yv[2][2][16];
#pragma unroll
  for (int pb = 0; pb < 2; ++pb) {
    const int px = pb * 32 + l32;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int c0 = wave * 64 + rb * 32 + hl * 16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 b = *reinterpret_cast<const f32x4*>(tb + c0 + 4 * i);
        const f32x4 s = *reinterpret_cast<const f32x4*>(tb + PR_N + c0 + 4 * i);
        const f32x4 r = *reinterpret_cast<const f32x4*>(lds + PR_RES + px * PR_RES_ROW + (((c0 >> 2) + i) ^ (px & 7)) * 16);
        // ((acc + bias) scale) + residual, each rounded (no fused multiply-add: the empty asm
        // pins the product), the LN-rows kernel's arithmetic, which adds the residual later
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float t = (acc[pb][rb][4 * i + e] + b[e]) * s[e];
          asm volatile("" : "+v"(t));
          yv[pb][rb][4 * i + e] = t + r[e];
        }
      }
      if constexpr (!CF32) {  // the rows are normalised from the stored (rounded) values
#pragma unroll
        for (int j = 0; j < 16; ++j) yv[pb][rb][j] = (float)(bf16_t)yv[pb][rb][j];
      }
    }
  }

  // ---- row statistics over the 512 channels, two passes as the reference: a lane's 32 values
  // in order, its pair lane (hl), the 8 waves in order through LDS
  float mean[2] = {0.f, 0.f}, rstd[2];
  const float invn = 1.0f / (float)PR_N;
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    if (pass == 0 && p.rms) continue;  // RMS: no centring
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
      float s = 0.f;
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const float d = pass == 0 ? yv[pb][rb][j] : yv[pb][rb][j] - mean[pb];
          s += pass == 0 ? d : d * d;
        }
      s += __shfl_xor(s, 32, 64);
      if (hl == 0) red[(pass * PR_WAVES + wave) * PR_P + pb * 32 + l32] = s;
    }
    barrier_keep_vm();
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < PR_WAVES; ++w) tot += red[(pass * PR_WAVES + w) * PR_P + pb * 32 + l32];
      if (pass == 0) mean[pb] = tot * invn;
      else rstd[pb] = rsqrtf(tot * invn + p.eps);
    }
  }

  // ---- normalised rows into LDS (over the residual, read by every wave before the barriers
  // above): pixel px, 16-byte unit u of its 64 at u ^ (px % 16)
#pragma unroll
  for (int pb = 0; pb < 2; ++pb) {
    const int px = pb * 32 + l32;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int c0 = wave * 64 + rb * 32 + hl * 16;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        f32x8 o;
#pragma unroll
        for (int i = 0; i < 8; ++i) o.v[i] = (yv[pb][rb][8 * h + i] - mean[pb]) * rstd[pb];
        const int u = (c0 >> 3) + h;
        *reinterpret_cast<bf16x8*>(lds + PR_ROWS + px * (PR_N * 2) + (u ^ (px & 15)) * 16) = pack_bf16(o);
      }
    }
  }
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.f;

  // ---- second GEMM: 8 waves x 64 W2^T rows per 512-row pass, A fragments from the LN rows, W2
  // fragments from L2 into registers one 64-k group ahead. The stores of this tile (y during
  // pass 0, each pass's out2 during the next pass) are spread over the groups, after the next
  // group's loads: the compiler's vmcnt waits before a group's MFMAs then leave them in flight
  // for two groups. Nothing in the loop branches around a memory instruction (the counts the
  // compiler derives at a join are those of the path with the fewest, which would wait for
  // every store): the stores are buffer stores bounded to the tile's valid rows (rows past M are
  // dropped by the range check), the look-ahead group index is clamped, and bias2 is read
  // through a range of 0 bytes when absent (zeros).
  int lane_f = lane, wave_f = wave;
  asm volatile("" : "+v"(lane_f), "+v"(wave_f));
  const int l32f = lane_f & 31, hlf = lane_f >> 5;
  const int npass = p.n2w / 512;
  const int total = npass * 8;  // 64-k groups
  constexpr int EC = CF32 ? 4 : 2;
  const int rows_ok = (int)(p.m - q0 < PR_P ? p.m - q0 : PR_P);
  const __amdgpu_buffer_rsrc_t yr = buf_rsrc_n((unsigned char*)p.c + q0 * p.ldc * EC, (uint32_t)(rows_ok * p.ldc * EC));
  const __amdgpu_buffer_rsrc_t ur =
      buf_rsrc_n((unsigned char*)p.out2 + q0 * p.ld2 * 2, (uint32_t)(rows_ok * p.ld2 * 2));
  const __amdgpu_buffer_rsrc_t br = buf_rsrc_n(p.bias2, p.bias2 ? (uint32_t)(p.n2w * 4) : 0u);
  // y store s of this lane: fp32, 16 of 16 bytes (block s / 4, elements 4 (s % 4) ..); bf16, 8 of
  // 16 bytes (block s / 2, elements 8 (s % 2) ..)
  constexpr int NY = CF32 ? 16 : 8;
  auto store_y = [&](const int s) __attribute__((always_inline)) {
    if constexpr (!CF32) {
      const int blk = s / 2, h = s % 2, pb = blk / 2, rb = blk % 2;
      const int c0 = wave_f * 64 + rb * 32 + hlf * 16 + 8 * h;
      f32x8 o;
#pragma unroll
      for (int i = 0; i < 8; ++i) o.v[i] = yv[pb][rb][8 * h + i];
      const bf16x8 ob = pack_bf16(o);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, ob), yr,
                                             (int)(((pb * 32 + l32f) * p.ldc + c0) * 2), 0, 0);
    } else {
      const int blk = s / 4, i = s % 4, pb = blk / 2, rb = blk % 2;
      const int c0 = wave_f * 64 + rb * 32 + hlf * 16 + 4 * i;
      const f32x4 v{yv[pb][rb][4 * i], yv[pb][rb][4 * i + 1], yv[pb][rb][4 * i + 2], yv[pb][rb][4 * i + 3]};
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), yr,
                                             (int)(((pb * 32 + l32f) * p.ldc + c0) * 4), 0, 0);
    }
  };
  const unsigned char* W2 = (const unsigned char*)p.w2p + ((int64_t)wave_f * 32 * 2 * 64 + lane_f) * 16;
  bf16x8 wf2[2][4][2];
  auto load_group = [&](int buf, int g) __attribute__((always_inline)) {
    const unsigned char* src = W2 + ((int64_t)(g / 8) * PR_WAVES * 32 * 2 + (g % 8) * 8) * 1024;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) wf2[buf][ks][rb] = *reinterpret_cast<const bf16x8*>(src + (ks * 2 + rb) * 1024);
  };
  load_group(0, 0);
  barrier_keep_vm();  // every wave's rows are in LDS
  auto group = [&](const int buf, const int g) __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int ua = (g % 8) * 8 + 2 * ks + hlf;
      bf16x8 af2[2];
#pragma unroll
      for (int pb = 0; pb < 2; ++pb) {
        const int px = pb * 32 + l32f;
        af2[pb] = *reinterpret_cast<const bf16x8*>(lds + PR_ROWS + px * (PR_N * 2) + (ua ^ (px & 15)) * 16);
      }
#pragma unroll
      for (int pb = 0; pb < 2; ++pb)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) acc[pb][rb] = mfma32_bf16(wf2[buf][ks][rb], af2[pb], acc[pb][rb]);
    }
  };
  // a pass's out2 through the wave's staging in row order (whole 128-byte row pieces; 64 bytes
  // with the gate): stage() writes the accumulators + bias2 (SimpleGate) rounded once to bf16,
  // store_u(pass, j) moves row group j (NST of them) to memory
  unsigned char* so = lds + PR_OUT + wave_f * 8192;
  constexpr int UPR = GATE ? 4 : 8;  // 16-byte units per staged row
  constexpr int PPI = 64 / UPR;      // rows per store
  constexpr int NST = PR_P / PPI;    // stores per pass
  // this lane's bias2 values of a pass: blocks (rb, i) at channel c0(rb) + 4 i; with the gate
  // rb = 0 / 1 are the two halves' columns of the same output channels
  f32x4 bv[2][4];
  auto chan = [&](const int pass, const int rb) __attribute__((always_inline)) {
    return GATE ? pass * 256 + wave_f * 32 + 16 * hlf + rb * (p.n2w / 2) : pass * 512 + wave_f * 64 + rb * 32 + 16 * hlf;
  };
  auto load_bias = [&](const int pass) __attribute__((always_inline)) {
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        bv[rb][i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(br, (chan(pass, rb) + 4 * i) * 4, 0, 0));
  };
  auto stage = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
      const int px = pb * 32 + l32f;
#pragma unroll
      for (int rb = 0; rb < (GATE ? 1 : 2); ++rb) {
        const int lc = GATE ? 16 * hlf : rb * 32 + 16 * hlf;
        float v[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (GATE) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              v[4 * i + e] = (acc[pb][0][4 * i + e] + bv[0][i][e]) * (acc[pb][1][4 * i + e] + bv[1][i][e]);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[4 * i + e] = acc[pb][rb][4 * i + e] + bv[rb][i][e];
          }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          f32x8 o;
#pragma unroll
          for (int i = 0; i < 8; ++i) o.v[i] = v[8 * h + i];
          const int u = lc / 8 + h;
          *reinterpret_cast<bf16x8*>(so + px * UPR * 16 + (u ^ (px & (UPR - 1))) * 16) = pack_bf16(o);
        }
      }
    }
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.f;
  };
  auto store_u = [&](const int pass, const int j) __attribute__((always_inline)) {
    const int c_base = GATE ? pass * 256 + wave_f * 32 : pass * 512 + wave_f * 64;
    const int px = j * PPI + lane_f / UPR, u = lane_f % UPR;
    const bf16x8 ov = *reinterpret_cast<const bf16x8*>(so + px * UPR * 16 + (u ^ (px & (UPR - 1))) * 16);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, ov), ur, (int)((px * p.ld2 + c_base + u * 8) * 2),
                                           0, 0);
  };
  // pass 0: per group, the next group's loads (the index clamped to the last group; before them,
  // two groups ahead of its use, the pass's bias2), the group's share of the y stores, then its
  // MFMAs
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (j == 6) load_bias(0);
    load_group((j + 1) & 1, j + 1 < total ? j + 1 : total - 1);
#pragma unroll
    for (int s = j * NY / 8; s < (j + 1) * NY / 8; ++s) store_y(s);
    __builtin_amdgcn_sched_barrier(0);  // the loads and stores go out before the MFMAs
    group(j & 1, j);
  }
  stage();
  // passes 1 .. npass - 1: the previous pass's out2 stores over the first NST groups
  for (int pass = 1; pass < npass; ++pass) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int g = pass * 8 + j;
      if (j == 6) load_bias(pass);
      load_group((j + 1) & 1, g + 1 < total ? g + 1 : total - 1);
      if (j < NST) store_u(pass - 1, j);
      __builtin_amdgcn_sched_barrier(0);
      group(j & 1, g);
    }
    stage();
  }
#pragma unroll
  for (int j = 0; j < NST; ++j) store_u(npass - 1, j);
  asm volatile("" ::"v"(touch[0]), "v"(touch[1]));
}

}  // namespace

}  // namespace clarus

using namespace clarus;

extern "C" int clarus_hip_gemm_ln_gemm_w1p(const ClarusGemmArgs* a, const void* w1p, float eps, int32_t rms,
                                           const void* w2p, const float* bias2, void* out2, int64_t n2w, int32_t gate2,
                                           void* stream) {
  clear_error();
  CLARUS_REQUIRE(a != nullptr && a->a && w1p && a->c && a->res && w2p && out2, "gemm_ln_gemm_w1p: null operand");
  CLARUS_REQUIRE(a->m > 0 && a->n == PR_N && a->k == PR_K, "gemm_ln_gemm_w1p: N = K = 512 (N=%lld K=%lld)",
                 (long long)a->n, (long long)a->k);
  CLARUS_REQUIRE(a->a_dtype == DT_BF16 && a->w_dtype == DT_BF16 && a->r_dtype == DT_F32 &&
                     (a->c_dtype == DT_BF16 || a->c_dtype == DT_F32),
                 "gemm_ln_gemm_w1p: bf16 A and W, fp32 residual, bf16 / fp32 output");
  CLARUS_REQUIRE(a->a_mode == CLARUS_A_ROWS && a->c_mode == CLARUS_C_ROWS && a->batch == 1 &&
                     (a->pro == PRO_NONE || a->pro == PRO_MUL) && !a->gate && a->act == ACT_NONE,
                 "gemm_ln_gemm_w1p: plain rows or the TLC-map prologue (no other prologue, gate, activation, "
                 "batch or pixel shuffle)");
  const bool mul = a->pro == PRO_MUL;
  if (mul) {
    CLARUS_REQUIRE(a->small && a->s_dtype == DT_BF16 && aligned(a->small, 16) && a->h > 0 && a->w > 0 && a->oh > 0 &&
                       a->ow > 0 && a->m % ((int64_t)a->h * a->w) == 0,
                   "gemm_ln_gemm_w1p: the map prologue needs a bf16 map (16-byte aligned) and m a multiple of h w");
  }
  const int ec = a->c_dtype == DT_BF16 ? 2 : 4;
  CLARUS_REQUIRE(a->lda >= a->k && (a->lda * 2) % 16 == 0 && aligned(a->a, 16) && aligned(w1p, 16) && aligned(w2p, 16),
                 "gemm_ln_gemm_w1p: 16-byte A rows and packed weights");
  CLARUS_REQUIRE(a->ldc >= a->n && (a->ldc * ec) % 16 == 0 && aligned(a->c, 16), "gemm_ln_gemm_w1p: 16-byte output rows");
  CLARUS_REQUIRE(a->ldr >= a->n && (a->ldr * 4) % 16 == 0 && aligned(a->res, 16), "gemm_ln_gemm_w1p: 16-byte residual rows");
  CLARUS_REQUIRE(aligned(out2, 16) && (bias2 == nullptr || aligned(bias2, 16)), "gemm_ln_gemm_w1p: 16-byte out2 / bias2");
  CLARUS_REQUIRE(eps >= 0.f && (rms == 0 || rms == 1), "gemm_ln_gemm_w1p: bad eps / mode");
  CLARUS_REQUIRE(n2w > 0 && n2w % 512 == 0 && n2w <= (1 << 20), "gemm_ln_gemm_w1p: n2w=%lld must be a multiple of 512",
                 (long long)n2w);
  CLARUS_REQUIRE(gate2 == 0 || gate2 == 1, "gemm_ln_gemm_w1p: gate2 is 0 or 1");
  CLARUS_REQUIRE(cdiv(a->m, PR_P) < ((int64_t)1 << 31), "gemm_ln_gemm_w1p: too many tiles");
  PairP p{};
  p.a = (const bf16_t*)a->a; p.w1p = w1p; p.bias = a->bias; p.scale = a->scale; p.res = (const float*)a->res;
  p.c = a->c; p.w2p = w2p; p.bias2 = bias2; p.out2 = out2;
  p.m = a->m; p.lda = a->lda; p.ldr = a->ldr; p.ldc = a->ldc; p.ld2 = gate2 ? n2w / 2 : n2w;
  p.c_dt = a->c_dtype; p.rms = rms; p.gate = gate2; p.n2w = (int)n2w;
  p.eps = eps; p.out_scale = a->out_scale;
  p.small = (const bf16_t*)a->small;
  p.h = a->h; p.w = a->w; p.oh = a->oh; p.ow = a->ow; p.pt = a->pt; p.pl = a->pl;
  note_kernel("pair_kernel gate=%d c=%s mul=%d", (int)gate2, a->c_dtype == DT_F32 ? "fp32" : "bf16", (int)mul);
  auto kern = mul ? (a->c_dtype == DT_F32 ? (gate2 ? pair_kernel<true, true, true> : pair_kernel<true, false, true>)
                                          : (gate2 ? pair_kernel<false, true, true> : pair_kernel<false, false, true>))
                  : (a->c_dtype == DT_F32 ? (gate2 ? pair_kernel<true, true, false> : pair_kernel<true, false, false>)
                                          : (gate2 ? pair_kernel<false, true, false> : pair_kernel<false, false, false>));
  static const bool attr = [] {
    for (auto k : {pair_kernel<true, true, false>, pair_kernel<true, false, false>, pair_kernel<false, true, false>,
                   pair_kernel<false, false, false>, pair_kernel<true, true, true>, pair_kernel<true, false, true>,
                   pair_kernel<false, true, true>, pair_kernel<false, false, true>})
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, PR_LDS);
    return true;
  }();
  (void)attr;
  hipLaunchKernelGGL(kern, dim3((unsigned)cdiv(a->m, PR_P)), dim3(PR_THREADS), PR_LDS, (hipStream_t)stream, p);
  return check_launch("gemm_ln_gemm_w1p");
}
