// Long-K bf16 GEMM with the weight streamed from L2 into registers: clarus_hip_gemm_wp (gfx950).
//
// y = act(A W^T + bias (SimpleGate: the product of both halves)) * scale * out_scale (+ residual)
// for plain bf16 rows A [m][K] (no prologue), K % 128 == 0, and W^T rows (N, or 2 N with the gate)
// a multiple of 512, with W^T also passed packed in the MFMA fragment order of
// clarus_hip_gemm_ln_gemm's second weight.
//
// Why: on the NAFNet level-2..4 shapes (M = 3600 .. 57600, K = 256 .. 1024) the LDS-staged tile
// kernels spend their K loop on LDS traffic (a 128 x 128 tile moves 32 KiB of copies and 64 KiB of
// fragment reads per 64-k chunk, about the MFMA time again) with one chunk in flight, and their
// epilogue reads the residual after the K loop, when every workgroup does so at once.
//
// One workgroup of 8 waves per (64-pixel tile, 512-row pass of W^T); wave w computes the 64 pixels
// x 64 W^T rows 64 w .. 64 w + 63 of the pass (2 x 2 blocks of 32x32x16 MFMAs, 64 accumulators):
//   * A chunks (64 rows x 64 k, 8 KiB) go global -> LDS by direct copies into a 3-stage ring
//     shared by the 8 waves, two chunks ahead; a chunk costs 8 KiB of copies and 64 KiB of
//     fragment reads;
//   * each wave's W^T fragments come from L2 straight into registers, packed so that one load
//     instruction moves 1 KiB of consecutive bytes, two 64-k groups (8 loads each) ahead: with one
//     group ahead the L2 round trip under this load (~1 us) exceeded a chunk's MFMA time and the
//     K loop took 1.2 - 1.8 us per chunk;
//   * the tile's residual (64 pixels x the pass's output channels) is copied into LDS during the
//     K loop, a few 1 KiB copies per chunk, so the epilogue reads it from LDS;
//   * epilogue in the MFMA layout: a lane holds 16 consecutive output channels of one pixel.
// Tiles are dealt XCD-aware: a contiguous range of (tile, pass) pairs per XCD, the passes of a
// pixel tile adjacent, so an A tile is fetched into one XCD's L2 once for all its passes.
// Without a residual two more forms: two passes per workgroup on one resident A tile (NPW = 2,
// once one pass per workgroup would need more than one round of the compute units) and
// wstream128_kernel (128-pixel tiles, K <= 512, while those still cover 3/4 of the units).
// Memory waits are explicit vmcnt counts: loads and copies complete in issue order.
// replaces kernels/gemm.py:353-400 (fused_gemm) for these shapes
#include <utility>

#include "capi.hpp"
#include "gemm_mfma32.hpp"

namespace clarus {

namespace {

constexpr int WS_P = 64, WS_WAVES = 8, WS_THREADS = 64 * WS_WAVES;
constexpr int WS_STAGE = WS_P * 128;                 // 8 KiB
constexpr int WS_STAGES = 3;
constexpr int WS_RES_MAX = WS_P * 512 * 4;           // 128 KiB: 64 rows x 512 fp32 channels
constexpr int WS_TB_FLOATS = 1024;                   // bias (512 W^T rows) + scale (<= 512 outputs)

__host__ __device__ constexpr int ws_res_row_bytes(bool gate, int rdt) {
  return rdt < 0 ? 0 : (gate ? 256 : 512) * (rdt == DT_F32 ? 4 : 2);
}
// A area: without a residual the whole A tile stays in LDS (NCH chunks), else the 3-stage ring
__host__ __device__ constexpr int ws_a_bytes(int rdt, int nch) { return (rdt < 0 ? nch : WS_STAGES) * WS_STAGE; }
// npw: W^T passes per workgroup, each with its own bias / scale table
__host__ __device__ constexpr int ws_lds_bytes(bool gate, int rdt, int nch, int npw) {
  return ws_a_bytes(rdt, nch) + WS_P * ws_res_row_bytes(gate, rdt) + npw * WS_TB_FLOATS * 4;
}
static_assert(ws_lds_bytes(false, DT_F32, 16, 1) <= 160 * 1024 && ws_lds_bytes(false, -1, 16, 2) <= 160 * 1024, "LDS");

struct WsP {
  const bf16_t* a;    // [m][lda]
  const void* wp;     // W^T packed: [pass][wave][16-k step][block][lane][8]
  const float* bias;  // [W^T rows] or null
  const float* scale; // [n] or null
  const void* res;    // [m][ldr] (RDT) or null
  void* c;            // [m][ldc] bf16 / fp32
  int64_t m, n, lda, ldr, ldc;
  int nch, npass, tiles, per_xcd;
  int c_dt, act;
  float out_scale, slope;
  float eps;  // LayerNorm / RMS prologue (wstream128_kernel)
  // map prologue (wstream_kernel with MUL): A row q times the bf16 map row of its pixel, the
  // map [n][oh][ow][K] replicate-padded to the h x w image by the offsets pt, pl
  const bf16_t* small;
  int h, w, oh, ow, pt, pl;
};

// RDT: residual dtype (-1: none); NCH: 64-k chunks (K / 64). The K loop is unrolled: with a
// run-time trip count the compiler's own wait insertion could not count the loads issued between
// a register's load and its use across the loop edge and drained every load before each chunk's
// first MFMA (vmcnt(0)), which undid the prefetch.
// NPW: consecutive W^T passes per workgroup (2 only without a residual). The pixel tile's A is
// copied into LDS once and serves both passes; the second pass's first two W^T groups are loaded
// before the first pass's epilogue, so its stores drain under the second pass's products, and the
// second pass needs no barrier (its A chunks are those the first pass already waited for).
// MUL (ring only): the map prologue of clarus_hip_rows_prologue applied to A in LDS. Each lane
// multiplies the 16-byte unit it copied of chunk c by the map values of its row, loaded at kernel
// start, once its own copies of the chunk have landed and before the barrier that publishes the
// chunk: widened to fp32, multiplied, rounded once to bf16, bit for bit the pass's rows.
template <bool GATE, int RDT, int NCH, int NPW, bool MUL>
__global__ void __launch_bounds__(WS_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
wstream_kernel(const WsP p) {
  constexpr int NO = GATE ? 256 : 512;                    // output channels per pass
  constexpr int RB = ws_res_row_bytes(GATE, RDT);         // residual bytes per row
  constexpr int CPW = RB / 128;                           // residual copies per wave (64 RB / 1 KiB / 8)
  constexpr int RSZ = RDT == DT_F32 ? 4 : 2;
  constexpr int RPC = CPW <= NCH ? 1 : (CPW <= 2 * NCH ? 2 : (CPW <= 4 * NCH ? 4 : 8));  // copies per chunk
  static_assert(CPW == 0 || (CPW % RPC == 0 && RPC * NCH >= CPW), "residual copies spread over the chunks");
  constexpr int nch = NCH;
  // Without a residual the A tile stays resident: chunks 0 .. 3 are copied in the prologue and
  // chunks c + 4, c + 5 in every even iteration c, so a barrier (to see the other waves' copies)
  // is needed only at even chunks. A barrier per chunk made every chunk wait for the slowest
  // wave's weight loads; larger batches held up the weight loads behind them (the wait counts
  // are in issue order).
  constexpr bool RESIDENT = RDT < 0;
  static_assert(NPW == 1 || (NPW == 2 && RESIDENT), "two passes per workgroup only with a resident A tile");
  static_assert(!MUL || (!RESIDENT && NCH <= 8), "the map prologue on the ring, K <= 512");
  constexpr int ABYTES = ws_a_bytes(RDT, NCH);
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  float* tb = reinterpret_cast<float*>(lds + ABYTES + WS_P * RB);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hl = lane >> 5;
  const int b = blockIdx.x;
  const int lin = (b & 7) * p.per_xcd + (b >> 3);
  if (lin >= p.tiles) return;  // before any LDS or memory traffic
  const int ngrp = p.npass / NPW;  // groups of NPW passes per pixel tile
  const int pt = lin / ngrp, ps0 = (lin - pt * ngrp) * NPW;
  const int64_t q0 = (int64_t)pt * WS_P;
  // ---- A chunk c (8 KiB): wave w copies rows 8 w .. 8 w + 7, lane l row 8 w + l / 8, slot l % 8
  const int arow = wave * 8 + (lane >> 3);
  int64_t aq = q0 + arow;
  if (aq > p.m - 1) aq = p.m - 1;  // rows past M: any valid row, never stored
  // ---- map values of this lane's unit in every chunk (the kernel's first memory operations: the
  // first chunk's wait covers them)
  u32x4 mv[MUL ? NCH : 1];
  if constexpr (MUL) {
    const int64_t hw = (int64_t)p.h * p.w;
    const int64_t im = aq / hw;
    const int rr = (int)(aq - im * hw);
    const int yq = rr / p.w;
    int sy = yq - p.pt, sx = rr - yq * p.w - p.pl;
    sy = sy < 0 ? 0 : (sy > p.oh - 1 ? p.oh - 1 : sy);
    sx = sx < 0 ? 0 : (sx > p.ow - 1 ? p.ow - 1 : sx);
    const bf16_t* mrow = p.small + ((im * p.oh + sy) * p.ow + sx) * (int64_t)(NCH * 64) + m32_swz(arow, lane & 7) * 8;
#pragma unroll
    for (int c = 0; c < NCH; ++c) mv[c] = *reinterpret_cast<const u32x4*>(mrow + c * 64);
    asm volatile("" ::: "memory");
  }

  // ---- the packed weight into this XCD's L2 first, when it fits comfortably (<= 2 MiB): the
  // XCD's workgroups read it all, in step, so from a cold cache each 64-k group would miss in all
  // of them at once. The per_xcd workgroups of an XCD each touch one 128-byte line in per_xcd (at
  // most two per thread; the index clamped, and line 0 only for a larger weight: no branch).
  // These are the kernel's first memory operations (the first chunk's wait covers them); the
  // values are consumed only at the end.
  unsigned int touch[2];
  {
    typedef const __attribute__((address_space(1))) unsigned int* gptr;
    const int64_t wbytes = (int64_t)p.npass * 512 * p.nch * 64 * 2;
    const bool on = wbytes <= ((int64_t)2 << 20);
    const int lines = (int)(wbytes / 128), slot = b >> 3;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      int l = (slot + i * p.per_xcd) * WS_THREADS + tid;
      l = !on ? 0 : (l < lines ? l : lines - 1);
      touch[i] = *(gptr)((const unsigned char*)p.wp + (int64_t)l * 128);
    }
  }
  asm volatile("" ::: "memory");
  const int64_t och0 = (int64_t)ps0 * NO;  // first output channel of the workgroup's first pass
  const unsigned char* asrc = (const unsigned char*)(p.a + aq * p.lda) + m32_swz(arow, lane & 7) * 16;
  auto issue_a = [&](int c) __attribute__((always_inline)) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(asrc + c * 128),
                                     (__attribute__((address_space(3))) void*)(lds + (RESIDENT ? c : c % WS_STAGES) * WS_STAGE + wave * 1024),
                                     16, 0, 0);
  };
  // ---- residual copy i of this wave: LDS bytes [1 KiB g, +1 KiB) of the rows, g = CPW w + i;
  // lane l lands at byte 1 KiB g + 16 l = row r, slot s, holding the row's 16-byte unit s ^ (r % 8)
  auto issue_res = [&](int c) __attribute__((always_inline)) {
    if constexpr (RDT >= 0) {
#pragma unroll
      for (int j = 0; j < RPC; ++j) {
        const int i = c * RPC + j;
        if (i < CPW) {
          const int off = (wave * CPW + i) * 1024 + lane * 16;
          const int r = off / RB, s = (off % RB) / 16;
          int64_t rq = q0 + r;
          if (rq > p.m - 1) rq = p.m - 1;
          const unsigned char* src =
              (const unsigned char*)p.res + (rq * p.ldr + och0) * RSZ + (s ^ (r & 7)) * 16;
          __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                           (__attribute__((address_space(3))) void*)(lds + ABYTES + (wave * CPW + i) * 1024),
                                           16, 0, 0);
        }
      }
    }
  };
  // ---- W^T group c (k 64 c .. 64 c + 63): 4 16-k steps x 2 blocks of this wave's 64 rows
  // (advanced by one pass, WS_WAVES * nch * 8 KiB, between the passes of an NPW = 2 workgroup)
  const unsigned char* wsrc =
      (const unsigned char*)p.wp + (((int64_t)ps0 * WS_WAVES + wave) * (nch * 4) * 2 * 64 + lane) * 16;
  bf16x8 wf[3][4][2];
  auto load_w = [&](int buf, int c) __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
        wf[buf][ks][rb] = *reinterpret_cast<const bf16x8*>(wsrc + ((int64_t)(4 * c + ks) * 2 + rb) * 1024);
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[x][y][j] = 0.f;

  // prologue: the tables of each pass (direct copies into LDS: bias of the pass's 512 W^T rows,
  // then scale of its output channels; 1 for a missing scale, 0 for a missing bias), A chunks 0
  // and 1, W^T groups 0 and 1
#pragma unroll
  for (int pi = 0; pi < NPW; ++pi) {
    const int64_t och = och0 + pi * NO;
    float* tp = tb + pi * WS_TB_FLOATS;
    const int64_t brow = GATE ? (wave < 4 ? och + 64 * wave : p.n + och + 64 * (wave - 4)) : och + 64 * wave;
    if (p.bias)
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(p.bias + brow + lane),
                                       (__attribute__((address_space(3))) void*)(tp + 64 * wave), 4, 0, 0);
    else
      tp[tid] = 0.f;
    if (64 * wave < NO) {
      if (p.scale)
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(p.scale + och + 64 * wave + lane),
                                         (__attribute__((address_space(3))) void*)(tp + 512 + 64 * wave), 4, 0, 0);
      else
        tp[512 + tid] = 1.f;
    }
  }
  asm volatile("" ::: "memory");
  issue_a(0);
  issue_a(1);
  if constexpr (RESIDENT) {
    issue_a(2);
    issue_a(3);
  }
  asm volatile("" ::: "memory");
  load_w(0, 0);
  asm volatile("" ::: "memory");
  load_w(1, 1);

  // chunk c from ring stage c % 3 and register buffer buf; with `next`, W^T group c + 2 is loaded
  // into buffer (buf + 2) % 3 two fragments per 16-k step, between the MFMAs, so that the vector
  // memory unit drains the workgroup's loads while the matrix cores run (issued all at once after
  // the barrier, the last wave's MFMAs started only once the others' loads had been accepted)
  auto chunk = [&](const int buf, const int c, const bool next) __attribute__((always_inline)) {
    const unsigned char* st = lds + (RESIDENT ? c : c % WS_STAGES) * WS_STAGE;
    const int nb = (buf + 2) % 3;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      bf16x8 af[2];
#pragma unroll
      for (int pb = 0; pb < 2; ++pb) {
        const int r = pb * 32 + l32;
        af[pb] = *reinterpret_cast<const bf16x8*>(st + r * 128 + m32_swz(r, 2 * ks + hl) * 16);
      }
      if (next) {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
          wf[nb][ks][rb] = *reinterpret_cast<const bf16x8*>(wsrc + ((int64_t)(4 * (c + 2) + ks) * 2 + rb) * 1024);
      }
      asm volatile("" ::: "memory");
#pragma unroll
      for (int pb = 0; pb < 2; ++pb)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) acc[pb][rb] = mfma32_bf16(wf[buf][ks][rb], af[pb], acc[pb][rb]);
    }
  };
  // Ring: iteration c issues A chunk c + 2, the residual copies of chunk c and W^T group c + 2, in
  // this order. Resident A: iteration c issues its A batch (if any), then W^T group c + 2. At the
  // top of iteration c A chunk c and W^T group c (W^T issued in iteration c - 2 after that A) must
  // have landed: still allowed outstanding is everything iteration c - 1 issued.
  auto res_copies = [&](int j) __attribute__((always_inline)) {
    return (RDT >= 0 && j >= 0 && j * RPC < CPW) ? RPC : 0;
  };
  auto batch_lo = [&](int c) __attribute__((always_inline)) { return c + 4 < NCH ? c + 4 : NCH; };
  auto batch_hi = [&](int c) __attribute__((always_inline)) {
    return c % 2 != 0 ? batch_lo(c) : (c + 6 < NCH ? c + 6 : NCH);
  };
  auto batch_n = [&](int c) __attribute__((always_inline)) {
    return c >= 0 && c % 2 == 0 && batch_hi(c) > batch_lo(c) ? batch_hi(c) - batch_lo(c) : 0;
  };
  auto step = [&](const int buf, const int c) __attribute__((always_inline)) {
    if (c == 0) {
      wait_vmcnt<8>();  // W^T group 1 outstanding (the tables and A chunks 0, 1 came before group 0)
    } else if constexpr (RESIDENT) {
      // the copies issued after W^T group c (exact after unrolling: 0, 1, 2 + 0 or 8)
      const int n = batch_n(c - 1) + (c + 1 < nch ? 8 : 0);
      if (n >= 10) wait_vmcnt<10>();
      else if (n >= 9) wait_vmcnt<9>();
      else if (n >= 8) wait_vmcnt<8>();
      else if (n >= 2) wait_vmcnt<2>();
      else if (n >= 1) wait_vmcnt<1>();
      else wait_vmcnt<0>();
    } else {
      // the largest allowed count that does not exceed the copies issued after W^T group c
      const int n = res_copies(c - 1) + (c + 1 < nch ? 9 : 0);
      if (n >= 9 + RPC) wait_vmcnt<9 + RPC>();
      else if (n >= 9) wait_vmcnt<9>();
      else if (n >= RPC) wait_vmcnt<RPC>();
      else wait_vmcnt<0>();
    }
    if constexpr (MUL) {  // this lane's unit of chunk c (its copy has landed) times the map
      unsigned char* up = lds + (c % WS_STAGES) * WS_STAGE + wave * 1024 + lane * 16;
      const u32x4 raw = *reinterpret_cast<const u32x4*>(up);
      f32x8 x;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x.v[2 * e] = __uint_as_float(raw[e] << 16) * __uint_as_float(mv[c][e] << 16);
        x.v[2 * e + 1] = __uint_as_float(raw[e] & 0xffff0000u) * __uint_as_float(mv[c][e] & 0xffff0000u);
      }
      *reinterpret_cast<bf16x8*>(up) = pack_bf16(x);
    }
    // ring: every wave's share of A chunk c, and chunk c - 1 read by all (its stage is refilled);
    // resident: every wave's share of the chunks up to the next batch
    if (!RESIDENT || c % 2 == 0) barrier_keep_vm();
    asm volatile("" ::: "memory");
    const bool next = c + 2 < nch;
    if constexpr (RESIDENT) {
#pragma unroll
      for (int j = batch_lo(c); j < batch_hi(c); ++j) issue_a(j);
    } else {
      if (next) issue_a(c + 2);
    }
    issue_res(c);
    asm volatile("" ::: "memory");
    chunk(buf, c, next);
  };

  // ---- epilogue of pass pi in the MFMA layout: block (pb, rb), lane (l32, hl): pixel
  // pb * 32 + l32; pass channel c0 = 64 wave + 32 rb + 16 hl (gate: 32 wave + 16 hl, both blocks)
  // .. c0 + 15
  auto epilogue = [&](const int pi) __attribute__((always_inline)) {
  const float* tt = tb + pi * WS_TB_FLOATS;  // the pass's tables
  const int64_t och = och0 + pi * NO;
#pragma unroll
  for (int pb = 0; pb < 2; ++pb) {
    const int px = pb * 32 + l32;
    const int64_t q = q0 + px;
#pragma unroll
    for (int rb = 0; rb < (GATE ? 1 : 2); ++rb) {
      const int c0 = GATE ? wave * 32 + hl * 16 : wave * 64 + rb * 32 + hl * 16;
      float v[16];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 b1 = *reinterpret_cast<const f32x4*>(tt + c0 + 4 * i);
        if constexpr (GATE) {
          const f32x4 b2 = *reinterpret_cast<const f32x4*>(tt + 256 + c0 + 4 * i);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[4 * i + e] = (acc[pb][0][4 * i + e] + b1[e]) * (acc[pb][1][4 * i + e] + b2[e]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[4 * i + e] = acc[pb][rb][4 * i + e] + b1[e];
        }
      }
      if (p.act == ACT_GELU) {
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = gelu_erf(v[j]);
      } else if (p.act == ACT_LRELU) {
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = v[j] >= 0.f ? v[j] : v[j] * p.slope;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 s = *reinterpret_cast<const f32x4*>(tt + 512 + c0 + 4 * i);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * i + e] *= s[e] * p.out_scale;
      }
      if constexpr (RDT == DT_F32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int u = (c0 >> 2) + i;
          const f32x4 r = *reinterpret_cast<const f32x4*>(lds + ABYTES + px * RB + (u ^ (px & 7)) * 16);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[4 * i + e] += r[e];
        }
      } else if constexpr (RDT == DT_BF16) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int u = (c0 >> 3) + i;
          const u32x4 r = *reinterpret_cast<const u32x4*>(lds + ABYTES + px * RB + (u ^ (px & 7)) * 16);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[8 * i + 2 * e] += __uint_as_float(r[e] << 16);
            v[8 * i + 2 * e + 1] += __uint_as_float(r[e] & 0xffff0000u);
          }
        }
      }
      if (q < p.m) {
        const int64_t o = q * p.ldc + och + c0;
        if (p.c_dt == DT_BF16) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            f32x8 ov;
#pragma unroll
            for (int i = 0; i < 8; ++i) ov.v[i] = v[8 * h + i];
            *reinterpret_cast<bf16x8*>((unsigned char*)p.c + (o + 8 * h) * 2) = pack_bf16(ov);
          }
        } else {
          float* op = reinterpret_cast<float*>(p.c) + o;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            reinterpret_cast<f32x4*>(op)[i] = f32x4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
        }
      }
    }
  }
  };

#pragma unroll
  for (int c = 0; c < NCH; ++c) step(c % 3, c);
  if constexpr (NPW == 1) {
    wait_vmcnt<0>();
    barrier_keep_vm();  // every residual row and the tables in LDS
    epilogue(0);
  } else {
    wsrc += (int64_t)WS_WAVES * nch * 8 * 1024;  // the second pass's W^T
    load_w(0, 0);
    asm volatile("" ::: "memory");
    load_w(1, 1);
    asm volatile("" ::: "memory");
    wait_vmcnt<16>();   // all but those two groups: the tables came first
    barrier_keep_vm();  // every wave's tables in LDS
    epilogue(0);
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int y = 0; y < 2; ++y)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[x][y][j] = 0.f;
    asm volatile("" ::: "memory");
#pragma unroll
    for (int c = 0; c < NCH; ++c) chunk(c % 3, c, c + 2 < NCH);
    epilogue(1);
  }
  asm volatile("" ::"v"(touch[0]), "v"(touch[1]));
}

// ---- 128-pixel tiles (no residual, K = 256 / 512) ------------------------------------------------
// With 64-pixel tiles the K loop is bound by the W^T stream from L2: each fragment feeds two MFMAs,
// and the second pass of a two-pass workgroup (no A copies, no barriers) still ran its 512-k loop at
// about 60 % of the MFMA rate. Here a wave keeps its 64 W^T rows' products for 128 pixels (4 x 2
// blocks of 32 x 32, 128 accumulator registers): every fragment feeds four MFMAs and the L2 bytes
// per product halve. W^T arrives one 16-k step (two fragments, 2 KiB per wave) at a time through a
// ring of W2_SLOTS register slots, W2_AHEAD steps ahead of its use (9 or 10 steps ran no faster).
// The A tile (128 pixels x K, 128 KiB at K = 512) is copied into LDS in the prologue and stays
// there. On the NAFNet level-3 shapes (M = 14400, K = 512, 226 workgroups) the K loop runs at
// about 83 % of the MFMA rate of the shader clock it gets under this load (s_memtime against
// s_memrealtime: 1.75 GHz, not the 2.4 GHz peak); the A fill before it (HBM) and the stores after
// it take the rest.
constexpr int W2_P = 128, W2_STAGE = W2_P * 128;  // 16 KiB per 64-k chunk
constexpr int W2_AHEAD = 7, W2_SLOTS = W2_AHEAD + 1;

__host__ __device__ constexpr int w2_lds_bytes(int nch) { return nch * W2_STAGE + WS_TB_FLOATS * 4; }
static_assert(w2_lds_bytes(8) <= 160 * 1024, "LDS");

// The prologue copies the whole A tile, then loads W^T steps 0 .. W2_AHEAD - 1 (two loads each);
// each step s then loads step s + W2_AHEAD. Loads and copies complete in issue order, so a copy
// queued ahead of a W^T load delays that load: copying chunk c + 2 at the top of chunk c tied every
// W^T load to an HBM round trip with less than two chunks of slack (1.8 us per 64-k chunk against
// 0.9 us of MFMA time). With outstanding copies the compiler's own wait insertion also stops
// counting (the copies write LDS): the first use of any register loaded before them drained the
// counter (vmcnt(0)) whatever the explicit waits. So the tile lands before the K loop (one wait,
// one barrier) and the loop waits on W^T loads only, with explicit counts:
// operations a wave has issued after its loads of W^T step t when step t's products start (after
// that step's load).
__host__ __device__ constexpr int w2_after_w(int t, int nch) {
  const int nt = 4 * nch, pre = W2_AHEAD < nt ? W2_AHEAD : nt;
  int n = 0, s0 = t - W2_AHEAD + 1;   // the first step after the one that loaded step t
  if (t < W2_AHEAD) {                 // loaded in the prologue
    n += 2 * (pre - 1 - t);
    s0 = 0;
  }
  for (int s = s0; s <= t; ++s)
    if (s + W2_AHEAD < nt) n += 2;
  return n;
}
static_assert(w2_after_w(0, 8) == 14 && w2_after_w(6, 8) == 14 && w2_after_w(7, 8) == 14 &&
                  w2_after_w(31, 8) == 0 && w2_after_w(24, 8) == 14 && w2_after_w(13, 4) == 4,
              "load counts");

template <class F, int... I>
__device__ __forceinline__ void unrolled(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}

// sum over the G lanes of a row group, butterfly in the order 1, 2, .. G / 2 (clarus_hip_rows_
// prologue's order, so the statistics below are bitwise those of that pass)
// PRO: PRO_NONE, or PRO_LN / PRO_RMS applied to whole rows (K <= 512) before the K loop: each row
// is normalised by one group of K / 8 lanes, lane g holding its k = 8 g .. 8 g + 7 as
// clarus_hip_rows_prologue does (two-pass statistics, the same butterfly, eps inside the square
// root) and rounded once to bf16, so the product sees the operand that pass would have written,
// bit for bit, without the pass's HBM round trip. ADT: the A rows' dtype: bf16 rows are copied
// into the LDS tile and normalised there; fp32 rows (the NAFNet trunk; 256 KiB a tile, more than
// LDS) are loaded into registers (all of a wave's rows at once, after the first W^T loads),
// normalised there and written to the tile as bf16.
template <bool GATE, int NCH, int PRO, int ADT>
__global__ void __launch_bounds__(WS_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
wstream128_kernel(const WsP p) {
  constexpr int NO = GATE ? 256 : 512;  // output channels per pass
  constexpr int NT = 4 * NCH;           // 16-k steps
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  float* tb = reinterpret_cast<float*>(lds + NCH * W2_STAGE);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hl = lane >> 5;
  const int b = blockIdx.x;
  const int lin = (b & 7) * p.per_xcd + (b >> 3);
  if (lin >= p.tiles) return;  // before any LDS or memory traffic

  // the packed weight into this XCD's L2 first, as in wstream_kernel
  unsigned int touch[2];
  {
    typedef const __attribute__((address_space(1))) unsigned int* gptr;
    const int64_t wbytes = (int64_t)p.npass * 512 * NCH * 64 * 2;
    const bool on = wbytes <= ((int64_t)2 << 20);
    const int lines = (int)(wbytes / 128), slot = b >> 3;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      int l = (slot + i * p.per_xcd) * WS_THREADS + tid;
      l = !on ? 0 : (l < lines ? l : lines - 1);
      touch[i] = *(gptr)((const unsigned char*)p.wp + (int64_t)l * 128);
    }
  }
  asm volatile("" ::: "memory");
  const int pt = lin / p.npass, ps = lin - pt * p.npass;
  const int64_t q0 = (int64_t)pt * W2_P;
  const int64_t och = (int64_t)ps * NO;  // first output channel of the pass

  // ---- A chunk c (16 KiB): copy j of wave w lands rows 16 w + 8 j .. + 7, lane l row
  // 16 w + 8 j + l / 8, slot l % 8 (holding the row's unit m32_swz(row, l % 8))
  const unsigned char* asrc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int arow = wave * 16 + j * 8 + (lane >> 3);
    int64_t aq = q0 + arow;
    if (aq > p.m - 1) aq = p.m - 1;  // rows past M: any valid row, never stored
    asrc[j] = (const unsigned char*)(p.a + aq * p.lda) + m32_swz(arow, lane & 7) * 16;
  }
  auto issue_a = [&](int c) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(asrc[j] + c * 128),
                                       (__attribute__((address_space(3))) void*)(lds + c * W2_STAGE + (2 * wave + j) * 1024),
                                       16, 0, 0);
  };
  // ---- W^T 16-k step t of this wave's 64 rows: 2 fragments (blocks) into ring slot t % W2_SLOTS
  const unsigned char* wsrc =
      (const unsigned char*)p.wp + (((int64_t)ps * WS_WAVES + wave) * NT * 2 * 64 + lane) * 16;
  bf16x8 wf[W2_SLOTS][2];
  auto load_w = [&](int t) __attribute__((always_inline)) {
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
      wf[t % W2_SLOTS][rb] = *reinterpret_cast<const bf16x8*>(wsrc + ((int64_t)t * 2 + rb) * 1024);
  };


  // prologue: the tables (bias of the pass's 512 W^T rows, then scale of its output channels; 0 /
  // 1 when left out), the A tile, the first W2_AHEAD W^T steps
  {
    const int64_t brow = GATE ? (wave < 4 ? och + 64 * wave : p.n + och + 64 * (wave - 4)) : och + 64 * wave;
    if (p.bias)
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(p.bias + brow + lane),
                                       (__attribute__((address_space(3))) void*)(tb + 64 * wave), 4, 0, 0);
    else
      tb[tid] = 0.f;
    if (64 * wave < NO) {
      if (p.scale)
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(p.scale + och + 64 * wave + lane),
                                         (__attribute__((address_space(3))) void*)(tb + 512 + 64 * wave), 4, 0, 0);
      else
        tb[512 + tid] = 1.f;
    }
  }
  asm volatile("" ::: "memory");
  constexpr bool REG_ROWS = PRO != PRO_NONE && ADT == DT_F32;  // fp32 rows through registers
  if constexpr (!REG_ROWS) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) issue_a(c);
    asm volatile("" ::: "memory");
  }
#pragma unroll
  for (int t = 0; t < (W2_AHEAD < NT ? W2_AHEAD : NT); ++t) {
    load_w(t);
    asm volatile("" ::: "memory");  // in step order: the wait counts below assume it
  }
  // ---- prologue geometry: a row is normalised by G = K / 8 lanes (RPW rows per wave at a time);
  // lane gl holds k = 8 gl .. 8 gl + 7, LDS unit un of chunk ch of the row
  constexpr int G = NCH * 8;
  constexpr int RPW = 64 / G;
  constexpr int NIT = W2_P / (WS_WAVES * RPW);  // rows per lane group of a wave
  const int sub = lane / G, gl = lane - sub * G;
  const int ch = gl >> 3, un = gl & 7;
  const float invk = 1.0f / (float)(NCH * 64);
  auto normalise = [&](f32x8& x) __attribute__((always_inline)) {
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
  };
  if constexpr (REG_ROWS) {
    // this wave's rows (wave RPW + 8 RPW it + sub), all loads in flight at once; rows past M
    // take row M - 1 (never stored)
    f32x8 xa[NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int r = wave * RPW + it * WS_WAVES * RPW + sub;
      int64_t aq = q0 + r;
      if (aq > p.m - 1) aq = p.m - 1;
      xa[it] = load8<DT_F32>(reinterpret_cast<const float*>(p.a) + aq * p.lda + 8 * gl);
    }
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int r = wave * RPW + it * WS_WAVES * RPW + sub;
      normalise(xa[it]);
      *reinterpret_cast<bf16x8*>(lds + ch * W2_STAGE + r * 128 + m32_swz(r, un) * 16) = pack_bf16(xa[it]);
    }
  }
  wait_vmcnt<2 * (W2_AHEAD < NT ? W2_AHEAD : NT)>();  // the tables and this wave's copies
  barrier_keep_vm();                                  // ... and every other wave's (or rows)
  if constexpr (PRO != PRO_NONE && !REG_ROWS) {
    for (int r0 = wave * RPW; r0 < W2_P; r0 += WS_WAVES * RPW) {
      const int r = r0 + sub;
      unsigned char* up = lds + ch * W2_STAGE + r * 128 + m32_swz(r, un) * 16;
      const u32x4 raw = *reinterpret_cast<const u32x4*>(up);
      f32x8 x;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x.v[2 * e] = __uint_as_float(raw[e] << 16);
        x.v[2 * e + 1] = __uint_as_float(raw[e] & 0xffff0000u);
      }
      normalise(x);
      *reinterpret_cast<bf16x8*>(up) = pack_bf16(x);
    }
    barrier_keep_vm();  // every row normalised
  }

  f32x16 acc[4][2];
#pragma unroll
  for (int x = 0; x < 4; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[x][y][j] = 0.f;

  // ---- K loop, unrolled over the 16-k steps (every wait count a constant)
  unrolled([&](auto tc) __attribute__((always_inline)) {
    constexpr int t = decltype(tc)::value;
    if constexpr (t + W2_AHEAD < NT) load_w(t + W2_AHEAD);
    asm volatile("" ::: "memory");
    wait_vmcnt<w2_after_w(t, NCH)>();  // this step's W^T fragments
    const unsigned char* st = lds + (t / 4) * W2_STAGE;
    bf16x8 af[4];
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
      const int r = pb * 32 + l32;
      af[pb] = *reinterpret_cast<const bf16x8*>(st + r * 128 + m32_swz(r, 2 * (t % 4) + hl) * 16);
    }
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int pb = 0; pb < 4; ++pb) acc[pb][rb] = mfma32_bf16(wf[t % W2_SLOTS][rb], af[pb], acc[pb][rb]);
  }, std::make_integer_sequence<int, NT>{});

  // ---- epilogue in the MFMA layout: block (pb, rb), lane (l32, hl): pixel pb * 32 + l32; pass
  // channel c0 = 64 wave + 32 rb + 16 hl (gate: 32 wave + 16 hl, both blocks) .. c0 + 15. The
  // tables landed before the K loop's wait and barrier.
#pragma unroll
  for (int pb = 0; pb < 4; ++pb) {
    const int64_t q = q0 + pb * 32 + l32;
#pragma unroll
    for (int rb = 0; rb < (GATE ? 1 : 2); ++rb) {
      const int c0 = GATE ? wave * 32 + hl * 16 : wave * 64 + rb * 32 + hl * 16;
      float v[16];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 b1 = *reinterpret_cast<const f32x4*>(tb + c0 + 4 * i);
        if constexpr (GATE) {
          const f32x4 b2 = *reinterpret_cast<const f32x4*>(tb + 256 + c0 + 4 * i);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[4 * i + e] = (acc[pb][0][4 * i + e] + b1[e]) * (acc[pb][1][4 * i + e] + b2[e]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[4 * i + e] = acc[pb][rb][4 * i + e] + b1[e];
        }
      }
      if (p.act == ACT_GELU) {
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = gelu_erf(v[j]);
      } else if (p.act == ACT_LRELU) {
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = v[j] >= 0.f ? v[j] : v[j] * p.slope;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 sc = *reinterpret_cast<const f32x4*>(tb + 512 + c0 + 4 * i);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * i + e] *= sc[e] * p.out_scale;
      }
      if (q < p.m) {
        const int64_t o = q * p.ldc + och + c0;
        if (p.c_dt == DT_BF16) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            f32x8 ov;
#pragma unroll
            for (int i = 0; i < 8; ++i) ov.v[i] = v[8 * h + i];
            *reinterpret_cast<bf16x8*>((unsigned char*)p.c + (o + 8 * h) * 2) = pack_bf16(ov);
          }
        } else {
          float* op = reinterpret_cast<float*>(p.c) + o;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            reinterpret_cast<f32x4*>(op)[i] = f32x4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
        }
      }
    }
  }
  asm volatile("" ::"v"(touch[0]), "v"(touch[1]));
}

template <bool GATE, int NCH, int PRO, int ADT>
void launch128(const WsP& p, hipStream_t s) {
  constexpr int lds = w2_lds_bytes(NCH);
  auto fn = &wstream128_kernel<GATE, NCH, PRO, ADT>;
  static const bool attr = [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    return true;
  }();
  (void)attr;
  hipLaunchKernelGGL(fn, dim3((unsigned)(8 * p.per_xcd)), dim3(WS_THREADS), lds, s, p);
}

template <int PRO, int ADT>
void launch128_g(const WsP& p, bool gate, hipStream_t s) {
  if (gate) {
    if (p.nch == 4) launch128<true, 4, PRO, ADT>(p, s);
    else launch128<true, 8, PRO, ADT>(p, s);
  } else {
    if (p.nch == 4) launch128<false, 4, PRO, ADT>(p, s);
    else launch128<false, 8, PRO, ADT>(p, s);
  }
}

template <bool GATE, int RDT, int NCH, int NPW, bool MUL = false>
void launch(const WsP& p, hipStream_t s) {
  constexpr int lds = ws_lds_bytes(GATE, RDT, NCH, NPW);
  auto fn = &wstream_kernel<GATE, RDT, NCH, NPW, MUL>;
  static const bool attr = [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    return true;
  }();
  (void)attr;
  hipLaunchKernelGGL(fn, dim3((unsigned)(8 * p.per_xcd)), dim3(WS_THREADS), lds, s, p);
}

template <bool GATE, int RDT>
void launch_k(const WsP& p, int npw, hipStream_t s, bool mul = false) {
  if constexpr (RDT >= 0) {
    if (mul) {
      if (p.nch == 4) launch<GATE, RDT, 4, 1, true>(p, s);
      else launch<GATE, RDT, 8, 1, true>(p, s);
      return;
    }
  }
  if constexpr (RDT < 0) {
    if (npw == 2) {
      if (p.nch == 4) launch<GATE, RDT, 4, 2>(p, s);
      else if (p.nch == 8) launch<GATE, RDT, 8, 2>(p, s);
      else launch<GATE, RDT, 16, 2>(p, s);
      return;
    }
  }
  if (p.nch == 4) launch<GATE, RDT, 4, 1>(p, s);
  else if (p.nch == 8) launch<GATE, RDT, 8, 1>(p, s);
  else launch<GATE, RDT, 16, 1>(p, s);
}

}  // namespace

}  // namespace clarus

using namespace clarus;

extern "C" int clarus_hip_gemm_wp(const ClarusGemmArgs* a, const void* wp, void* stream) {
  clear_error();
  CLARUS_REQUIRE(a != nullptr && a->a && wp && a->c, "gemm_wp: null operand");
  const int pro = a->pro;
  const bool gate = a->gate != 0;
  const int64_t nw = gate ? 2 * a->n : a->n;
  CLARUS_REQUIRE(a->m > 0 && a->n > 0 && nw % 512 == 0 && (a->k == 256 || a->k == 512 || a->k == 1024),
                 "gemm_wp: W^T rows a multiple of 512, K = 256, 512 or 1024 (N=%lld K=%lld gate=%d)",
                 (long long)a->n, (long long)a->k, (int)gate);
  CLARUS_REQUIRE((a->a_dtype == DT_BF16 || (a->a_dtype == DT_F32 && pro != PRO_NONE)) && a->w_dtype == DT_BF16 &&
                     (a->c_dtype == DT_BF16 || a->c_dtype == DT_F32),
                 "gemm_wp: bf16 A (fp32 with a prologue) and W, bf16 / fp32 output");
  CLARUS_REQUIRE(a->res == nullptr || a->r_dtype == DT_BF16 || a->r_dtype == DT_F32, "gemm_wp: bf16 / fp32 residual");
  // a LayerNorm / RMS prologue (no residual, K <= 512) runs inside the 128-pixel kernel, on the
  // whole rows its A tile holds; the map prologue (a residual, K <= 512, bf16 A and map) on the
  // 64-pixel ring's chunks
  const bool mul = pro == PRO_MUL;
  CLARUS_REQUIRE(pro == PRO_NONE || ((pro == PRO_LN || pro == PRO_RMS) && a->res == nullptr && a->k <= 512) ||
                     (mul && a->res != nullptr && a->k <= 512),
                 "gemm_wp: no prologue, LayerNorm / RMS without a residual at K <= 512, or the map prologue "
                 "with a residual at K <= 512 (pro=%d)", pro);
  if (mul) {
    CLARUS_REQUIRE(a->small && a->s_dtype == DT_BF16 && a->a_dtype == DT_BF16 && aligned(a->small, 16) &&
                       a->h > 0 && a->w > 0 && a->oh > 0 && a->ow > 0 && a->m % ((int64_t)a->h * a->w) == 0,
                   "gemm_wp: the map prologue needs a bf16 map (16-byte aligned), bf16 A and m a multiple of h w");
  }
  CLARUS_REQUIRE(a->a_mode == CLARUS_A_ROWS && a->c_mode == CLARUS_C_ROWS && a->batch == 1 &&
                     (a->act == ACT_NONE || a->act == ACT_GELU || a->act == ACT_LRELU),
                 "gemm_wp: plain rows (no batch or pixel shuffle)");
  const int ec = a->c_dtype == DT_BF16 ? 2 : 4;
  const int ea = a->a_dtype == DT_F32 ? 4 : 2;
  CLARUS_REQUIRE(a->lda >= a->k && (a->lda * ea) % 16 == 0 && aligned(a->a, 16) && aligned(wp, 16),
                 "gemm_wp: 16-byte A rows and packed weight");
  CLARUS_REQUIRE(a->ldc >= a->n && (a->ldc * ec) % 16 == 0 && aligned(a->c, 16), "gemm_wp: 16-byte output rows");
  if (a->res) {
    const int rs = a->r_dtype == DT_BF16 ? 2 : 4;
    CLARUS_REQUIRE(a->ldr >= a->n && (a->ldr * rs) % 16 == 0 && aligned(a->res, 16), "gemm_wp: 16-byte residual rows");
  }
  const int64_t ptiles = cdiv(a->m, WS_P), npass = nw / 512;
  CLARUS_REQUIRE(ptiles * npass < ((int64_t)1 << 30), "gemm_wp: too many tiles");
  // two W^T passes per workgroup (no residual, an even pass count) once one pass per workgroup
  // would take more than one round of the device's compute units: A is then read once and the
  // second round's A fill and epilogue are gone
  const int npw = a->res == nullptr && npass % 2 == 0 && ptiles * npass > device_cus() ? 2 : 1;
  // 128-pixel tiles (half the L2 weight bytes per product) without a residual at K <= 512, while
  // their (tile, pass) count still covers at least 3/4 of the compute units
  const int64_t ptiles128 = cdiv(a->m, W2_P);
  const bool p128 = a->res == nullptr && a->k <= 512 &&
                    (pro != PRO_NONE || 4 * ptiles128 * npass >= 3 * (int64_t)device_cus());
  WsP p{};
  p.a = (const bf16_t*)a->a; p.wp = wp; p.bias = a->bias; p.scale = a->scale; p.res = a->res; p.c = a->c;
  p.m = a->m; p.n = a->n; p.lda = a->lda; p.ldr = a->ldr; p.ldc = a->ldc;
  p.nch = (int)(a->k / 64); p.npass = (int)npass;
  p.tiles = (int)(p128 ? ptiles128 * npass : ptiles * npass / npw);
  p.per_xcd = (int)cdiv(p.tiles, 8);
  p.c_dt = a->c_dtype; p.act = a->act; p.out_scale = a->out_scale; p.slope = a->slope; p.eps = a->ln_eps;
  p.small = (const bf16_t*)a->small;
  p.h = (int)a->h; p.w = (int)a->w; p.oh = (int)a->oh; p.ow = (int)a->ow; p.pt = (int)a->pt; p.pl = (int)a->pl;
  const int rdt = a->res ? a->r_dtype : -1;
  note_kernel("wstream_kernel gate=%d res=%d pro=%d k=%lld p=%d npw=%d", (int)gate, rdt, pro, (long long)a->k,
              p128 ? W2_P : WS_P, p128 ? 1 : npw);
  hipStream_t s = (hipStream_t)stream;
  if (p128) {
    const bool f32 = a->a_dtype == DT_F32;
    if (pro == PRO_LN) f32 ? launch128_g<PRO_LN, DT_F32>(p, gate, s) : launch128_g<PRO_LN, DT_BF16>(p, gate, s);
    else if (pro == PRO_RMS) f32 ? launch128_g<PRO_RMS, DT_F32>(p, gate, s) : launch128_g<PRO_RMS, DT_BF16>(p, gate, s);
    else launch128_g<PRO_NONE, DT_BF16>(p, gate, s);
  } else if (gate) {
    if (rdt == DT_F32) launch_k<true, DT_F32>(p, npw, s, mul);
    else if (rdt == DT_BF16) launch_k<true, DT_BF16>(p, npw, s, mul);
    else launch_k<true, -1>(p, npw, s);
  } else {
    if (rdt == DT_F32) launch_k<false, DT_F32>(p, npw, s, mul);
    else if (rdt == DT_BF16) launch_k<false, DT_BF16>(p, npw, s, mul);
    else launch_k<false, -1>(p, npw, s);
  }
  return check_launch("gemm_wp");
}
