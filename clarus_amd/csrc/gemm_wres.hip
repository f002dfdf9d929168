// Short-K bf16 GEMM with the weight resident in registers, persistent over pixel tiles:
// clarus_hip_gemm_wr (gfx950).
//
// y = act(A W^T + bias (SimpleGate: the product of both halves)) * scale * out_scale (+ residual)
// for plain bf16 rows A [m][K], K = 128 or 256, with W^T passed packed in the fragment order of
// clarus_hip_gemm_wp (passes of 512 W^T rows; with the gate each half padded to 256 rows, without
// it the rows padded to a multiple of 512, the padding zero).
//
// Why: at K <= 256 a 64-pixel tile is only 1 - 2 us of MFMA work, and the tile kernels spend
// as long again waiting for their first chunk and writing their output (NAFNet level 2 / config-2
// c256: 900 single-tile workgroups ran in four rounds of ~6 us, of which the K loop was 2 us).
//
// One workgroup of 8 waves per CU (persistent), one 512-row W^T pass per workgroup: wave w keeps
// the pass's W^T rows 64 w .. 64 w + 63 for all of K in registers (K / 16 steps x 2 blocks of
// 32 rows, 64 or 128 VGPRs), loaded once, and computes 64 pixels x those 64 rows per tile (2 x 2
// blocks of 32x32x16 MFMAs). Waves whose rows are all padding skip the products and stores.
//   * A tiles (64 rows x K, 16 / 32 KiB) travel global -> LDS by direct copies into two buffers:
//     the next tile's copies are issued at the top of a tile, so they land during its K loop and
//     epilogue. A rows are 2K bytes with their 16-byte units XOR-swizzled by row % 16 (the 16
//     lanes reading one unit of 16 consecutive rows hit distinct bank groups);
//   * the tile's residual (64 pixels x the pass's output channels, <= 64 KiB) is copied into LDS
//     at the top of the tile and read by the epilogue;
//   * epilogue in the MFMA layout (a lane holds 16 consecutive output channels of one pixel) with
//     buffer stores bounded to the tile's valid rows, so every wave issues the same number of
//     stores and the wait at the next tile's top can leave them in flight.
// A pass with at most 256 real W^T rows (N <= 256, or N <= 128 with the gate) leaves waves 4 - 7
// holding padding; HALF then gives wave w + 4 the rows of wave w and splits the tile's pixels
// between them (wave w: pixels 0 .. 31, wave w + 4: 32 .. 63), so every SIMD runs two working
// waves and one wave's epilogue overlaps the other's products (the same sums, bit for bit).
// Workgroups go to the XCDs in turn (XCD = block % 8); each XCD owns a contiguous range of pixel
// tiles and its workgroups split into the passes, so an A tile is fetched into one L2 for all of
// its passes. Memory waits are explicit vmcnt counts (copies, loads and stores complete in issue
// order for the counter).
// replaces kernels/gemm.py:353-400 (fused_gemm) for these shapes
#include "capi.hpp"
#include "gemm_mfma32.hpp"

namespace clarus {

namespace {

constexpr int WR_P = 64, WR_WAVES = 8, WR_THREADS = 64 * WR_WAVES;
constexpr int WR_TB_FLOATS = 1024;  // bias of the pass's 512 W^T rows, scale of its outputs

__host__ __device__ constexpr int wr_res_row_bytes(int rc, int rdt) {
  return rdt < 0 ? 0 : rc * (rdt == DT_F32 ? 4 : 2);
}
// A buffers: two (the next tile's copies land during the current tile)
__host__ __device__ constexpr int wr_nbuf(int) { return 2; }
__host__ __device__ constexpr int wr_lds_bytes(int k, int rc, int rdt) {
  return wr_nbuf(rdt) * WR_P * k * 2 + WR_P * wr_res_row_bytes(rc, rdt) + WR_TB_FLOATS * 4;
}
static_assert(wr_lds_bytes(256, 256, DT_F32) <= 160 * 1024 && wr_lds_bytes(256, 512, DT_BF16) <= 160 * 1024 &&
                  wr_lds_bytes(256, 0, -1) <= 160 * 1024, "LDS");

struct WrP {
  const bf16_t* a;    // [m][lda]
  const void* wp;     // W^T packed: [pass][wave][16-k step][block][lane][8]
  const float* bias;  // [n] or [2 n] with the gate, or null
  const float* scale; // [n] or null
  const void* res;    // [m][ldr] or null
  void* c;            // [m][ldc]
  int64_t m, n, lda, ldr, ldc;
  int npass, ptiles, act;
  float out_scale, slope, eps;
  // PRO_MUL: A row q times the bf16 map row of its pixel ([n][oh][ow][K], replicate-padded to the
  // h x w image by the offsets pt, pl)
  const bf16_t* small;
  int h, w, oh, ow, pt, pl;
};

// GATE: SimpleGate pairs (256 output channels per pass); RDT: residual dtype (-1 none); CDT:
// output dtype; K: 128 or 256; RC: residual channels staged per row (256, or 512 without the gate);
// HALF: one pass of at most 256 real W^T rows, its pixels split over wave pairs; PRO: PRO_NONE,
// PRO_LN / PRO_RMS applied to the A tile's rows in LDS before its products (no residual), or PRO_MUL
// (no gate): each lane multiplies the units it copied of a tile by their map values (loaded just
// before the tile's copies, so they land first) once its copies have landed, before the barrier
// that publishes the tile; widened to fp32, multiplied, rounded once to bf16 as the separate pass
template <bool GATE, int RDT, int CDT, int K, int RC, bool HALF, int PRO>
__global__ void __launch_bounds__(WR_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
wres_kernel(const WrP p) {
  constexpr int KS = K / 16;                 // 16-k steps
  constexpr int ROWB = K * 2;                // bytes per A row in LDS
  constexpr int ABYTES = WR_P * ROWB;        // one A buffer
  constexpr int NA = ABYTES / 1024 / WR_WAVES;  // A copies per wave (2 or 4)
  constexpr int NO = GATE ? 256 : 512;       // output channels per pass
  constexpr int RSZ = RDT == DT_F32 ? 4 : 2;
  constexpr int RB = wr_res_row_bytes(RC, RDT);
  constexpr int NR = RDT < 0 ? 0 : WR_P * RB / 1024 / WR_WAVES;  // residual copies per wave
  constexpr int OES = CDT == DT_F32 ? 4 : 2;
  constexpr int NPB = HALF ? 1 : 2;          // 32-pixel blocks per wave and tile
  constexpr int NS = NPB * (GATE ? 1 : 2) * (16 * OES / 16);  // 16-byte stores per lane per tile
  static_assert(RDT < 0 || (WR_P * RB) % (1024 * WR_WAVES) == 0, "residual copies per wave");
  static_assert(RDT < 0 || RC >= NO || !GATE, "the gate stages all 256 channels");
  static_assert(PRO == PRO_NONE || PRO == PRO_MUL || RDT < 0, "a row prologue only without a residual");
  static_assert(PRO != PRO_MUL || !GATE, "the map prologue without the gate");
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  constexpr int NBUF = wr_nbuf(RDT);
  unsigned char* rbuf = lds + NBUF * ABYTES;
  float* tb = reinterpret_cast<float*>(rbuf + WR_P * RB);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  // ---- which pass and tiles: XCD x = block % 8 owns pixel tiles [x T / 8, (x + 1) T / 8); its
  // workgroups j = block / 8 split into the passes (j % npass) and walk the range with stride R
  const int nblk = (int)gridDim.x;
  const int x = blockIdx.x & 7, j = blockIdx.x >> 3, J = nblk >> 3;
  const int pass = j % p.npass, R = J / p.npass, r0 = j / p.npass;
  if (r0 >= R) return;  // a leftover workgroup (J not a multiple of npass), before any memory traffic
  const int t_lo = (int)((int64_t)x * p.ptiles / 8), t_hi = (int)((int64_t)(x + 1) * p.ptiles / 8);
  const int t_first = t_lo + r0;
  if (t_first >= t_hi) return;
  const int64_t och = (int64_t)pass * NO;  // first output channel of the pass
  // waves whose 64 W^T rows (32 output channels with the gate) are all padding
  const int wrow = HALF ? (wave & 3) : wave;  // the wave whose W^T rows this wave holds
  const bool active = (GATE ? och + 32 * wrow : och + 64 * wrow) < p.n;
  const bool scaled = p.scale != nullptr || p.out_scale != 1.f;  // else the scale table is all 1

  // ---- this wave's W^T fragments of the pass, all of K, into registers
  bf16x8 wf[KS][2];
  {
    const unsigned char* wsrc = (const unsigned char*)p.wp + (((int64_t)pass * WR_WAVES + wrow) * KS * 2 * 64 + lane) * 16;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int b = 0; b < 2; ++b) wf[s][b] = *reinterpret_cast<const bf16x8*>(wsrc + ((int64_t)s * 2 + b) * 1024);
  }
  asm volatile("" ::: "memory");

  // ---- copies. A tile t into buffer bf: copy g = NA w + i moves LDS bytes [1 KiB g, +1 KiB):
  // lane l lands at row (1024 g + 16 l) / ROWB, slot s, and holds the row's unit s ^ (row % 16)
  auto issue_a = [&](int t, int bf, int lane, int wave) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int off = (wave * NA + i) * 1024 + lane * 16;
      const int row = off / ROWB, s = (off % ROWB) / 16;
      int64_t q = (int64_t)t * WR_P + row;
      if (q > p.m - 1) q = p.m - 1;  // rows past M: any valid row, never stored
      const unsigned char* src = (const unsigned char*)(p.a + q * p.lda) + (s ^ (row & 15)) * 16;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                       (__attribute__((address_space(3))) void*)(lds + bf * ABYTES + (wave * NA + i) * 1024),
                                       16, 0, 0);
    }
  };
  // residual of tile t: row r, slot s holds the row's unit s ^ (r % 8)
  auto issue_r = [&](int t, int lane, int wave) __attribute__((always_inline)) {
    if constexpr (RDT >= 0) {
#pragma unroll
      for (int i = 0; i < NR; ++i) {
        const int off = (wave * NR + i) * 1024 + lane * 16;
        const int row = off / RB, s = (off % RB) / 16;
        int64_t q = (int64_t)t * WR_P + row;
        if (q > p.m - 1) q = p.m - 1;
        const unsigned char* src = (const unsigned char*)p.res + (q * p.ldr + och) * RSZ + (s ^ (row & 7)) * 16;
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                         (__attribute__((address_space(3))) void*)(rbuf + (wave * NR + i) * 1024),
                                         16, 0, 0);
      }
    }
  };

  // map values of the units this lane copies of tile t (the row and unit of issue_a's copy i)
  u32x4 mv[PRO == PRO_MUL ? NA : 1];
  auto load_map = [&](int t, int lane, int wave) __attribute__((always_inline)) {
    if constexpr (PRO == PRO_MUL) {
      const int64_t hw = (int64_t)p.h * p.w;
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        const int off = (wave * NA + i) * 1024 + lane * 16;
        const int row = off / ROWB, s = (off % ROWB) / 16;
        int64_t q = (int64_t)t * WR_P + row;
        if (q > p.m - 1) q = p.m - 1;
        const int64_t im = q / hw;
        const int rr = (int)(q - im * hw);
        const int yq = rr / p.w;
        int sy = yq - p.pt, sx = rr - yq * p.w - p.pl;
        sy = sy < 0 ? 0 : (sy > p.oh - 1 ? p.oh - 1 : sy);
        sx = sx < 0 ? 0 : (sx > p.ow - 1 ? p.ow - 1 : sx);
        mv[i] = *reinterpret_cast<const u32x4*>(p.small + ((im * p.oh + sy) * p.ow + sx) * (int64_t)K +
                                                (s ^ (row & 15)) * 8);
      }
    }
  };

  f32x16 acc[NPB][2];
  load_map(t_first, lane, wave);
  asm volatile("" ::: "memory");
  issue_a(t_first, 0, lane, wave);
  // ---- tables (after the W^T loads and the first copies, so the three latencies overlap): bias of the pass's W^T rows (gate: the first halves' 256, then the second
  // halves'), scale of its output channels (1 for none, 0 bias for none; 0 past n)
  {
    const int c = tid;  // 512 threads, one table entry each
    const int64_t ch = GATE ? och + (c & 255) : och + c;
    const int64_t brow = GATE ? (c < 256 ? ch : p.n + ch) : ch;
    tb[c] = (p.bias && ch < p.n) ? p.bias[brow] : 0.f;
    if (c < NO) tb[512 + c] = ((p.scale && och + c < p.n) ? p.scale[och + c] : 1.f) * p.out_scale;
  }
  // ---- LayerNorm / RMS of the rows of the A tile in buffer bf, in place, in clarus_hip_rows_
  // prologue's order: a row is normalised by G = K / 8 consecutive lanes, lane gl holding its
  // k = 8 gl .. 8 gl + 7 (the row's unit gl, at slot gl ^ (row % 16)); two-pass statistics, the
  // same butterfly, eps inside the square root; rounded once to bf16. The products then see the
  // operand that pass would have written, bit for bit, without its round trip through HBM.
  auto normalise_tile = [&](const int bf, const int ln, const int wv) __attribute__((always_inline)) {
    constexpr int G = K / 8, RPW = 64 / G;  // lanes per row, rows per wave at a time
    const int sub = ln / G, gl = ln - sub * G;
    const float invk = 1.0f / (float)K;
    unsigned char* ab = lds + bf * ABYTES;
#pragma unroll
    for (int r0 = 0; r0 < WR_P; r0 += WR_WAVES * RPW) {
      const int r = r0 + wv * RPW + sub;
      unsigned char* up = ab + r * ROWB + (gl ^ (r & 15)) * 16;
      const u32x4 raw = *reinterpret_cast<const u32x4*>(up);
      f32x8 x;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x.v[2 * e] = __uint_as_float(raw[e] << 16);
        x.v[2 * e + 1] = __uint_as_float(raw[e] & 0xffff0000u);
      }
      float mean = 0.f;
      if constexpr (PRO == PRO_LN) {
        float sm = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) sm += x.v[i];
        mean = group_sum<G>(sm) * invk;
      }
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float d = x.v[i] - mean;
        ss += d * d;
      }
      const float rstd = rsqrtf(group_sum<G>(ss) * invk + p.eps);
#pragma unroll
      for (int i = 0; i < 8; ++i) x.v[i] = (x.v[i] - mean) * rstd;
      *reinterpret_cast<bf16x8*>(up) = pack_bf16(x);
    }
  };
  // ---- one tile: the products of A(t) from buffer bf into acc, then its epilogue
  // pixel block i of this wave: i, or with HALF the wave pair's half ph
  auto kloop = [&](const int bf, const int l32, const int hl, const int ph) __attribute__((always_inline)) {
#pragma unroll
  for (int a = 0; a < NPB; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;
  if (active) {
    // A fragments one 16-k step ahead of the MFMAs (the scheduling barriers keep the reads of
    // later steps from being hoisted, which would take a register per read)
    const unsigned char* ab = lds + bf * ABYTES;
    bf16x8 af[2][NPB];
    auto read_a = [&](int s, int buf) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < NPB; ++i) {
        const int row = (HALF ? ph : i) * 32 + l32;
        af[buf][i] = *reinterpret_cast<const bf16x8*>(ab + row * ROWB + ((2 * s + hl) ^ (row & 15)) * 16);
      }
    };
    read_a(0, 0);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if (s + 1 < KS) read_a(s + 1, (s + 1) & 1);
#pragma unroll
      for (int i = 0; i < NPB; ++i)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) acc[i][rb] = mfma32_bf16(wf[s][rb], af[s & 1][i], acc[i][rb]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  };
  auto epilogue = [&](const int t, const int l32, const int hl, const int wave) __attribute__((always_inline)) {
  // ---- epilogue: block (pb, rb), lane (l32, hl): pixel pb * 32 + l32; pass channel c0 =
  // 64 wave + 32 rb + 16 hl (gate: 32 wave + 16 hl, both blocks) .. c0 + 15
  const int64_t q0 = (int64_t)t * WR_P;
  const int rows_ok = (int)(p.m - q0 < WR_P ? p.m - q0 : WR_P);
  const int nval = (int)(p.n - och < NO ? p.n - och : NO);  // output channels of the pass
  const __amdgpu_buffer_rsrc_t cr =
      buf_rsrc_n((unsigned char*)p.c + (q0 * p.ldc + och) * OES, (uint32_t)((rows_ok - 1) * p.ldc * OES + nval * OES));
  const int wr = HALF ? (wave & 3) : wave, ph = wave >> 2;  // row-owning wave, pixel half
  if (active) {
#pragma unroll
    for (int ib = 0; ib < NPB; ++ib) {
      const int pb = HALF ? ph : ib;
      const int px = pb * 32 + l32;
#pragma unroll
      for (int rb = 0; rb < (GATE ? 1 : 2); ++rb) {
        const int c0 = GATE ? wr * 32 + hl * 16 : wr * 64 + rb * 32 + hl * 16;
        float v[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x4 b1 = *reinterpret_cast<const f32x4*>(tb + c0 + 4 * i);
          if constexpr (GATE) {
            const f32x4 b2 = *reinterpret_cast<const f32x4*>(tb + 256 + c0 + 4 * i);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[4 * i + e] = (acc[ib][0][4 * i + e] + b1[e]) * (acc[ib][1][4 * i + e] + b2[e]);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[4 * i + e] = acc[ib][rb][4 * i + e] + b1[e];
          }
        }
        if (p.act == ACT_GELU) {
#pragma unroll
          for (int e = 0; e < 16; ++e) v[e] = gelu_erf(v[e]);
        } else if (p.act == ACT_LRELU) {
#pragma unroll
          for (int e = 0; e < 16; ++e) v[e] = v[e] >= 0.f ? v[e] : v[e] * p.slope;
        }
        if (scaled) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const f32x4 s = *reinterpret_cast<const f32x4*>(tb + 512 + c0 + 4 * i);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[4 * i + e] *= s[e];
          }
        }
        if constexpr (RDT == DT_F32) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int u = (c0 >> 2) + i;
            const f32x4 rv = *reinterpret_cast<const f32x4*>(rbuf + px * RB + (u ^ (px & 7)) * 16);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[4 * i + e] += rv[e];
          }
        } else if constexpr (RDT == DT_BF16) {
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const int u = (c0 >> 3) + i;
            const u32x4 rv = *reinterpret_cast<const u32x4*>(rbuf + px * RB + (u ^ (px & 7)) * 16);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              v[8 * i + 2 * e] += __uint_as_float(rv[e] << 16);
              v[8 * i + 2 * e + 1] += __uint_as_float(rv[e] & 0xffff0000u);
            }
          }
        }
        // rows past M start past the range (ldc >= n); a run past n (the padding of the last
        // pass) is sent past it too, so every lane still issues every store
        const bool keep = och + c0 < p.n;
        const int o = (int)((px * p.ldc + c0) * OES);
        if constexpr (CDT == DT_BF16) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            f32x8 ov;
#pragma unroll
            for (int i = 0; i < 8; ++i) ov.v[i] = v[8 * h + i];
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, pack_bf16(ov)), cr,
                                                   keep ? o + 16 * h : 0x7ffffff0, 0, 0);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_raw_buffer_store_b128(
                __builtin_bit_cast(u32x4, f32x4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]}), cr,
                keep ? o + 16 * i : 0x7ffffff0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);  // one block's temporaries live at a time
      }
    }
  }
  };
  // the lane and wave indices laundered per tile: the addresses derived from them are then
  // recomputed per tile instead of being hoisted out of the loop and held in registers
  auto fresh = [&](int& ln, int& wv) __attribute__((always_inline)) {
    ln = threadIdx.x & 63;
    wv = threadIdx.x >> 6;
    asm volatile("" : "+v"(ln), "+v"(wv));
  };

  // One barrier at the top of a tile: every wave's copies of A(t) have landed and every wave is
  // done with the previous tile (its A buffer, and the residual buffer its epilogue read, are
  // free). A third A buffer, or the barrier between a tile's products and its epilogue, measured
  // no faster: the two waves of a SIMD then wait on each other's products instead.
  int bf = 0;
  for (int t = t_first; t < t_hi; t += R, bf ^= 1) {
    int ln, wv;
    fresh(ln, wv);
    const int l32 = ln & 31, hl = ln >> 5;
    const bool has_next = t + R < t_hi;
    // this wave's copies of A(t) have landed (what was issued after them: the previous tile's
    // stores; a wave without outputs issues none), then every wave's
    if (t == t_first || !active) wait_vmcnt<0>();
    else wait_vmcnt<NS>();
    if constexpr (PRO == PRO_MUL) {  // this lane's units of A(t) (its copies have landed) times the map
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        unsigned char* up = lds + bf * ABYTES + (wv * NA + i) * 1024 + ln * 16;
        const u32x4 raw = *reinterpret_cast<const u32x4*>(up);
        f32x8 xm;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          xm.v[2 * e] = __uint_as_float(raw[e] << 16) * __uint_as_float(mv[i][e] << 16);
          xm.v[2 * e + 1] = __uint_as_float(raw[e] & 0xffff0000u) * __uint_as_float(mv[i][e] & 0xffff0000u);
        }
        *reinterpret_cast<bf16x8*>(up) = pack_bf16(xm);
      }
    }
    barrier_keep_vm();
    asm volatile("" ::: "memory");
    issue_r(t, ln, wv);
    if (has_next) {
      load_map(t + R, ln, wv);  // before the copies: landed when they have
      asm volatile("" ::: "memory");
      issue_a(t + R, bf ^ 1, ln, wv);
    }
    asm volatile("" ::: "memory");
    if constexpr (PRO == PRO_LN || PRO == PRO_RMS) {
      normalise_tile(bf, ln, wv);
      barrier_keep_vm();  // every row of the tile normalised
      asm volatile("" ::: "memory");
    }
    kloop(bf, l32, hl, wv >> 2);
    // the residual copies (issued before the next tile's A copies) have landed, in every wave
    if constexpr (RDT >= 0) {
      if (has_next) wait_vmcnt<NA>();
      else wait_vmcnt<0>();
      barrier_keep_vm();
      asm volatile("" ::: "memory");
    }
    epilogue(t, l32, hl, wv);
    asm volatile("" ::: "memory");
  }
}

template <bool GATE, int RDT, int CDT, int K, int RC, bool HALF, int PRO>
void launch(const WrP& p, int nblk, hipStream_t s) {
  constexpr int lds = wr_lds_bytes(K, RC, RDT);
  auto fn = &wres_kernel<GATE, RDT, CDT, K, RC, HALF, PRO>;
  static const bool attr = [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    return true;
  }();
  (void)attr;
  hipLaunchKernelGGL(fn, dim3((unsigned)nblk), dim3(WR_THREADS), lds, s, p);
}

template <bool GATE, int RDT, int CDT, int RC, int PRO>
void launch_k(const WrP& p, int k, bool half, int nblk, hipStream_t s) {
  if (half) {
    if (k == 128) launch<GATE, RDT, CDT, 128, RC, true, PRO>(p, nblk, s);
    else launch<GATE, RDT, CDT, 256, RC, true, PRO>(p, nblk, s);
  } else {
    if (k == 128) launch<GATE, RDT, CDT, 128, RC, false, PRO>(p, nblk, s);
    else launch<GATE, RDT, CDT, 256, RC, false, PRO>(p, nblk, s);
  }
}

// the map prologue: at K = 256 the half-pass form only (the full-pass forms with it spill)
template <int RDT, int CDT, int RC>
void launch_mul_k(const WrP& p, int k, bool half, int nblk, hipStream_t s) {
  if (k == 128) {
    if (half) launch<false, RDT, CDT, 128, RC, true, PRO_MUL>(p, nblk, s);
    else launch<false, RDT, CDT, 128, RC, false, PRO_MUL>(p, nblk, s);
  } else {
    launch<false, RDT, CDT, 256, RC, true, PRO_MUL>(p, nblk, s);
  }
}

template <int RDT, int RC>
void launch_mul(const WrP& p, int cdt, int k, bool half, int nblk, hipStream_t s) {
  if (cdt == DT_F32) launch_mul_k<RDT, DT_F32, RC>(p, k, half, nblk, s);
  else launch_mul_k<RDT, DT_BF16, RC>(p, k, half, nblk, s);
}

template <bool GATE, int RDT, int RC, int PRO = PRO_NONE>
void launch_c(const WrP& p, int cdt, int k, bool half, int nblk, hipStream_t s) {
  if (cdt == DT_F32) launch_k<GATE, RDT, DT_F32, RC, PRO>(p, k, half, nblk, s);
  else launch_k<GATE, RDT, DT_BF16, RC, PRO>(p, k, half, nblk, s);
}

}  // namespace

}  // namespace clarus

using namespace clarus;

extern "C" int clarus_hip_gemm_wr(const ClarusGemmArgs* a, const void* wp, void* stream) {
  clear_error();
  CLARUS_REQUIRE(a != nullptr && a->a && wp && a->c, "gemm_wr: null operand");
  const bool gate = a->gate != 0;
  CLARUS_REQUIRE(a->m > 0 && a->n > 0 && (a->k == 128 || a->k == 256) && a->n % 16 == 0,
                 "gemm_wr: K = 128 or 256, N a multiple of 16 (N=%lld K=%lld)", (long long)a->n, (long long)a->k);
  CLARUS_REQUIRE(a->a_dtype == DT_BF16 && a->w_dtype == DT_BF16 && (a->c_dtype == DT_BF16 || a->c_dtype == DT_F32),
                 "gemm_wr: bf16 A and W, bf16 / fp32 output");
  CLARUS_REQUIRE(a->res == nullptr || a->r_dtype == DT_BF16 || a->r_dtype == DT_F32, "gemm_wr: bf16 / fp32 residual");
  CLARUS_REQUIRE(a->a_mode == CLARUS_A_ROWS && a->c_mode == CLARUS_C_ROWS && a->batch == 1 &&
                     (a->act == ACT_NONE || a->act == ACT_GELU || a->act == ACT_LRELU),
                 "gemm_wr: plain rows (no batch or pixel shuffle)");
  // a LayerNorm / RMS prologue on the A tile's rows in LDS, without a residual; the map prologue
  // without the gate
  const int pro = a->pro;
  CLARUS_REQUIRE(pro == PRO_NONE || ((pro == PRO_LN || pro == PRO_RMS) && a->res == nullptr) ||
                     (pro == PRO_MUL && !gate),
                 "gemm_wr: no prologue, LayerNorm / RMS without a residual, or the map prologue without the gate "
                 "(pro=%d)", pro);
  if (pro == PRO_MUL) {
    CLARUS_REQUIRE(a->small && a->s_dtype == DT_BF16 && aligned(a->small, 16) && a->h > 0 && a->w > 0 && a->oh > 0 &&
                       a->ow > 0 && a->m % ((int64_t)a->h * a->w) == 0,
                   "gemm_wr: the map prologue needs a bf16 map (16-byte aligned) and m a multiple of h w");
  }
  const int ec = a->c_dtype == DT_BF16 ? 2 : 4;
  CLARUS_REQUIRE(a->lda >= a->k && (a->lda * 2) % 16 == 0 && aligned(a->a, 16) && aligned(wp, 16),
                 "gemm_wr: 16-byte A rows and packed weight");
  CLARUS_REQUIRE(a->ldc >= a->n && (a->ldc * ec) % 16 == 0 && aligned(a->c, 16), "gemm_wr: 16-byte output rows");
  const int64_t no = gate ? 256 : 512;
  const int64_t npass = cdiv(a->n, no);
  int rc = 0;
  if (a->res) {
    const int rs = a->r_dtype == DT_BF16 ? 2 : 4;
    CLARUS_REQUIRE(a->ldr >= a->n && (a->ldr * rs) % 16 == 0 && aligned(a->res, 16), "gemm_wr: 16-byte residual rows");
    // staged residual rows [och, och + rc) of every pass lie inside [0, n): rc = 256 with the gate
    // (N a multiple of 256) or for N = 256, 128 for N = 128 (bf16, no gate), else 512 (bf16, N a
    // multiple of 512)
    rc = (!gate && a->n == 128) ? 128 : ((gate || a->n <= 256) ? 256 : 512);
    CLARUS_REQUIRE(a->n % rc == 0 && (rc == 256 || a->r_dtype == DT_BF16),
                   "gemm_wr: a residual needs N a multiple of 256 with the gate, N = 256, or a bf16 residual "
                   "with N = 128 or a multiple of 512");
  }
  const int64_t ptiles = cdiv(a->m, WR_P);
  CLARUS_REQUIRE(ptiles < ((int64_t)1 << 30) && a->m * a->ldc * ec < ((int64_t)1 << 40), "gemm_wr: too many tiles");
  CLARUS_REQUIRE((WR_P - 1) * a->ldc * ec + no * ec < ((int64_t)1 << 31), "gemm_wr: output rows too long");
  const int cus = device_cus();
  int nblk = 8 * (cus / 8);
  if (nblk < 8 * (int)npass) nblk = 8 * (int)npass;
  WrP p{};
  p.a = (const bf16_t*)a->a; p.wp = wp; p.bias = a->bias; p.scale = a->scale; p.res = a->res; p.c = a->c;
  p.m = a->m; p.n = a->n; p.lda = a->lda; p.ldr = a->ldr; p.ldc = a->ldc;
  p.npass = (int)npass; p.ptiles = (int)ptiles; p.act = a->act; p.out_scale = a->out_scale; p.slope = a->slope;
  p.eps = a->ln_eps;
  p.small = (const bf16_t*)a->small;
  p.h = a->h; p.w = a->w; p.oh = a->oh; p.ow = a->ow; p.pt = a->pt; p.pl = a->pl;
  const int rdt = a->res ? a->r_dtype : -1;
  // one pass with at most 256 real W^T rows: waves 4 - 7 take the pixel halves (HALF)
  const bool half = npass == 1 && (gate ? a->n <= 128 : a->n <= 256);
  note_kernel("wres_kernel gate=%d res=%d k=%lld half=%d pro=%d", (int)gate, rdt, (long long)a->k, (int)half, pro);
  hipStream_t s = (hipStream_t)stream;
  const int k = (int)a->k, cdt = a->c_dtype;
  if (pro == PRO_MUL) {
    CLARUS_REQUIRE(k == 128 || half, "gemm_wr: the map prologue at K = 256 needs N <= 256 (one half pass)");
    if (rdt == DT_F32) launch_mul<DT_F32, 256>(p, cdt, k, half, nblk, s);
    else if (rdt == DT_BF16 && rc == 128) launch_mul<DT_BF16, 128>(p, cdt, k, half, nblk, s);
    else if (rdt == DT_BF16 && rc == 512) launch_mul<DT_BF16, 512>(p, cdt, k, half, nblk, s);
    else if (rdt == DT_BF16) launch_mul<DT_BF16, 256>(p, cdt, k, half, nblk, s);
    else launch_mul<-1, 256>(p, cdt, k, half, nblk, s);
  } else if (pro != PRO_NONE) {
    if (gate) {
      if (pro == PRO_LN) launch_c<true, -1, 256, PRO_LN>(p, cdt, k, half, nblk, s);
      else launch_c<true, -1, 256, PRO_RMS>(p, cdt, k, half, nblk, s);
    } else {
      if (pro == PRO_LN) launch_c<false, -1, 256, PRO_LN>(p, cdt, k, half, nblk, s);
      else launch_c<false, -1, 256, PRO_RMS>(p, cdt, k, half, nblk, s);
    }
  } else if (gate) {
    if (rdt == DT_F32) launch_c<true, DT_F32, 256>(p, cdt, k, half, nblk, s);
    else if (rdt == DT_BF16) launch_c<true, DT_BF16, 256>(p, cdt, k, half, nblk, s);
    else launch_c<true, -1, 256>(p, cdt, k, half, nblk, s);
  } else {
    if (rdt == DT_F32) launch_c<false, DT_F32, 256>(p, cdt, k, half, nblk, s);
    else if (rdt == DT_BF16 && rc == 128) launch_c<false, DT_BF16, 128>(p, cdt, k, half, nblk, s);
    else if (rdt == DT_BF16 && rc == 512) launch_c<false, DT_BF16, 512>(p, cdt, k, half, nblk, s);
    else if (rdt == DT_BF16) launch_c<false, DT_BF16, 256>(p, cdt, k, half, nblk, s);
    else launch_c<false, -1, 256>(p, cdt, k, half, nblk, s);
  }
  return check_launch("gemm_wr");
}
