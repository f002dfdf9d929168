// Mamba selective scan of EVSSM (one direction, no z gate, d_state 8) on gfx950.
//
// For crop t, channel d and state n along the raster sequence l = 0 .. L - 1:
//   delta_l = softplus(dt_raw_l . dt_w[d] + dt_bias[d])
//   h_l[n]  = 2^(delta_l a2[d, n]) h_{l-1}[n] + delta_l B_l[n] u_l[d]      (a2 = A log2(e))
//   y_l[d]  = sum_n C_l[n] h_l[n] + D[d] u_l[d]
// with dbl_l = [dt_raw (r) | B (8) | C (8) | ...] fp32 (row stride nc), u bf16 or fp32, y fp32.
//
// One lane per channel, one wave per (crop, SPW segments, CPW channels) with SPW * CPW = 64
// (CPW = 32 when d is not a multiple of 64, so d = 96 wastes no lanes): the 8 states live in
// registers and every step is a handful of FMAs and 8 exp2. A step's dbl row is the same for
// all lanes of a segment. Loads run one chunk of CH steps ahead: the chunk's u values go to
// registers, its dbl rows to LDS (B and C at fixed slots, dt_raw after them), so the recurrence
// waits on memory once per chunk, not once per step. The sequence is cut into segments so that
// enough waves run:
//   1. scan_kernel<SUMMARY>: per segment from h = 0, its end state and sum(delta)
//   2. carry_kernel:         along the segments of a crop, each segment's start state
//                            H0[s] = decay(s - 1) H0[s - 1] + E[s - 1], decay = 2^(a2 sum delta)
//   3. scan_kernel<final>:   per segment from H0[s], writing y
// (1 and 2 are skipped for a single segment.) The decay of a long segment can be far below
// fp32's normal range while decay * state is not: it is applied as
// 2^max(ld, -126) * (h * 2^min(ld + 126, 0)), exact to rounding for ld >= -252 and below that
// smaller than |h| 2^-252. Every sum runs in a fixed order: deterministic.
// replaces python/clarus/kernels/ssm.py:28-190 (scan8_kernel, carry_kernel, selective_scan)
#include <math.h>

#include "capi.hpp"
#include "common.hpp"

namespace clarus {

namespace {

constexpr int NS = 8;   // d_state
constexpr int MAXR = 16;

struct ScanP {
  const void* u;       // [t, l, d]
  const float* dbl;    // [t, l, nc]
  const float* dtw;    // [d, r]
  const float* dtb;    // [d]
  const float* a2;     // [d, 8]
  const float* dsk;    // [d]
  float* y;            // [t, l, d]
  float* dsum;         // [t, nseg, d]
  float* eh;           // [t, nseg, 8, d] end states from h = 0
  float* h0;           // [t, nseg, 8, d] start states
  int64_t t, l, d, nc, seg, nseg;
  int r;
};

// softplus(x) = ln(1 + e^x) (x for x > 20, as torch's threshold), from the hardware exp2 / log2:
// ln(1 + e) = log2(u) ln2 * e / (u - 1) with u = fl(1 + e) (Kahan's log1p: the factor e / (u - 1)
// undoes the rounding of 1 + e, so small e keeps full relative accuracy)
__device__ __forceinline__ float softplus(float x) {
  const float e = __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
  const float u = 1.0f + e;
  const float lp = u == 1.0f ? e : __builtin_amdgcn_logf(u) * 0.6931471805599453f * (e * __builtin_amdgcn_rcpf(u - 1.0f));
  return x > 20.0f ? x : lp;
}

constexpr int CH = 16;   // steps per chunk (a multiple of 2: rows are loaded two per instruction)
constexpr int RW = 32;   // LDS row: B (8) | C (8) | dt_raw (up to 16)

// dbl column held in LDS slot lc: B, C first (fixed offsets for 16-byte reads), then dt_raw
__device__ __forceinline__ int lds_col_src(int lc, int r) { return lc < 2 * NS ? r + lc : lc - 2 * NS; }

template <int UDT, bool SUMMARY, bool HAS_H0, int CPW>
__global__ void __launch_bounds__(64) scan_kernel(const ScanP p) {
  constexpr int SPW = 64 / CPW;
  constexpr int SUBF = CH * RW + 4;  // floats per segment's chunk in LDS (+4: other bank group)
  __shared__ __align__(16) float rows[2][SPW * SUBF];
  const int lane = threadIdx.x;
  const int sub = lane / CPW, cl = lane % CPW;
  const int64_t d = (int64_t)blockIdx.y * CPW + cl;
  const bool dv = d < p.d;
  const int64_t dl = dv ? d : 0;
  const int64_t nts = p.t * p.nseg;
  const int64_t ts_raw = (int64_t)blockIdx.x * SPW + sub;  // crop * nseg + segment
  const bool tv = ts_raw < nts;
  const int64_t ts = tv ? ts_raw : nts - 1;  // idle lanes shadow the last segment, write nothing
  const bool wr = dv && tv;
  const int64_t t = ts / p.nseg, s = ts - t * p.nseg;
  const int64_t l0 = s * p.seg;
  const int nsteps = (int)((l0 + p.seg < p.l ? l0 + p.seg : p.l) - l0);
  // the wave's shortest segment (SPW = 2: lanes 0 and 63 are in different segments)
  const int nmin = min(__shfl(nsteps, 0), __shfl(nsteps, 63));
  const int nch = (int)((p.seg + CH - 1) / CH);

  float w[MAXR];
#pragma unroll
  for (int i = 0; i < MAXR; ++i) w[i] = i < p.r ? p.dtw[dl * p.r + i] : 0.f;
  const float bias = p.dtb[dl];
  float a[NS], h[NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    a[n] = p.a2[dl * NS + n];
    h[n] = HAS_H0 ? p.h0[(ts * NS + n) * p.d + dl] : 0.f;
  }
  const float dskip = SUMMARY ? 0.f : p.dsk[dl];
  float dsum = 0.f;

  // a chunk's dbl rows reach LDS by direct copies: copy j moves elements j * 64 .. + 63 of the
  // wave's SPW x CH x RW block (row = e / RW, slot = e % RW); slots holding no dbl column keep
  // the zeros written below (their lanes copy nothing)
  constexpr int NJ = SPW * CH * RW / 64;
  const int lc = lane % RW;
  const bool col_ok = lc < 2 * NS || lc - 2 * NS < p.r;
  const int64_t colc = col_ok ? lds_col_src(lc, p.r) : 0;
  int64_t rbase[SPW];  // row index of each of the wave's segments' first step, and its step count
  int rlen[SPW];
#pragma unroll
  for (int q = 0; q < SPW; ++q) {
    int64_t tq = (int64_t)blockIdx.x * SPW + q;
    tq = tq < nts ? tq : nts - 1;
    const int64_t ct = tq / p.nseg, cs = tq - ct * p.nseg;
    rbase[q] = ct * p.l + cs * p.seg;
    rlen[q] = (int)((cs * p.seg + p.seg < p.l ? cs * p.seg + p.seg : p.l) - cs * p.seg);
  }
  constexpr int UES = UDT == DT_BF16 ? 2 : 4;
  const unsigned char* ub = (const unsigned char*)p.u + ((t * p.l + l0) * p.d + dl) * UES;
  float* yp = p.y + (t * p.l + l0) * p.d + dl;

  for (int i = lane; i < 2 * SPW * SUBF; i += 64) (&rows[0][0])[i] = 0.f;
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

  float uc[CH], un[CH];
  const int64_t ustr = p.d * UES;
  auto load_u = [&](const unsigned char* q) {
    return UDT == DT_BF16 ? bf16_to_f32(*reinterpret_cast<const unsigned short*>(q)) : *reinterpret_cast<const float*>(q);
  };
  auto load_chunk = [&](int c, int buf, float (&uo)[CH]) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      // copy j: segment q = j * 64 / (CH * RW), rows row0 .. row0 + 64 / RW - 1 of its chunk
      const int q = (j * 64) / (CH * RW), row0 = ((j * 64) % (CH * RW)) / RW;
      const int lim = rlen[q] - 1 - c * CH;  // the segment's last row, relative to the chunk
      const int row = row0 + lane / RW;
      const int rr = row < lim ? row : lim;
      const float* base = p.dbl + (rbase[q] + c * CH) * p.nc;  // uniform
      if (col_ok)
        __builtin_amdgcn_global_load_lds(
            (const __attribute__((address_space(1))) void*)(base + (rr * p.nc + colc)),
            (__attribute__((address_space(3))) void*)(&rows[buf][q * SUBF + (j * 64) % (CH * RW)]), 4, 0, 0);
    }
    const unsigned char* uq = ub + (int64_t)(c * CH) * ustr;
    if ((c + 1) * CH <= nmin) {
#pragma unroll
      for (int k = 0; k < CH; ++k) uo[k] = load_u(uq + k * ustr);
    } else {
      const int lim = nsteps - 1 - c * CH;
#pragma unroll
      for (int k = 0; k < CH; ++k) uo[k] = load_u(uq + (k < lim ? k : lim) * ustr);
    }
  };

  load_chunk(0, 0, uc);
  for (int c = 0; c < nch; ++c) {
    const int buf = c & 1;
    // chunk c's copies (issued one chunk ago) have landed; the other buffer's reads are done
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    barrier_keep_vm();
    if (c + 1 < nch) load_chunk(c + 1, buf ^ 1, un);
    const float* rw = &rows[buf][sub * SUBF];
    const bool full = (c + 1) * CH <= nmin;
    float* yc = yp + (int64_t)(c * CH) * p.d;
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      if (!(full || c * CH + k < nsteps)) continue;  // past this lane's segment end (last chunk)
      const float4* r4 = reinterpret_cast<const float4*>(rw + k * RW);
      const float4 b0 = r4[0], b1 = r4[1];
      float acc = bias;
#pragma unroll
      for (int i4 = 0; i4 < MAXR / 4; ++i4) {
        if (4 * i4 < p.r) {
          const float4 dt = r4[4 + i4];
          acc = fmaf(dt.x, w[4 * i4], acc);
          acc = fmaf(dt.y, w[4 * i4 + 1], acc);
          acc = fmaf(dt.z, w[4 * i4 + 2], acc);
          acc = fmaf(dt.w, w[4 * i4 + 3], acc);
        }
      }
      const float delta = softplus(acc);
      const float uv = uc[k];
      const float du = delta * uv;
      const float bb[NS] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
      // 2^(delta a) <= 1; a result below fp32's normal range is flushed, an error under 2^-126 |h|
      for (int n = 0; n < NS; ++n) h[n] = fmaf(__builtin_amdgcn_exp2f(delta * a[n]), h[n], du * bb[n]);
      if (SUMMARY) {
        dsum += delta;
      } else {
        const float4 c0 = r4[2], c1 = r4[3];
        const float cc[NS] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
        float yv = dskip * uv;
#pragma unroll
        for (int n = 0; n < NS; ++n) yv += h[n] * cc[n];
        if (wr) yc[k * p.d] = yv;
      }
    }
    if (c + 1 < nch) {
#pragma unroll
      for (int k = 0; k < CH; ++k) uc[k] = un[k];
    }
  }
  if (SUMMARY && wr) {
    p.dsum[ts * p.d + d] = dsum;
#pragma unroll
    for (int n = 0; n < NS; ++n) p.eh[(ts * NS + n) * p.d + d] = h[n];
  }
}

// one thread per (crop, state, channel): the segments' start states in order. The chain's inputs
// (sum delta and end state of each segment) do not depend on it: they are loaded CB segments at a
// time, the next batch in flight while the current one runs, so the chain waits on memory once
// per batch. (Loaded inside the chain, after the previous segment's store that the compiler
// could not tell apart from them, every step waited a full memory round trip: 342 segments of the
// EVSSM level-0 scan took 179 us.) 2 CB loads per batch: the next batch's stay within the 63
// loads a wait count can leave in flight.
constexpr int CB = 16;

__global__ void __launch_bounds__(256) carry_kernel(const ScanP p) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // n * d + channel
  const int64_t t = blockIdx.y;
  if (i >= NS * p.d) return;
  const int64_t n = i / p.d, d = i - n * p.d;
  const float a = p.a2[d * NS + n];
  const int64_t nseg = p.nseg, sd = p.d, se = NS * p.d;  // strides between segments
  const float* __restrict__ dsum = p.dsum + t * nseg * sd + d;
  const float* __restrict__ eh = p.eh + (t * nseg * NS + n) * sd + d;
  // start states through the crop's range (a wave-uniform descriptor, the lane's element in the
  // offset): the stores of the padding segments of the last batch go past the range and are
  // dropped, so every batch issues the same loads and stores (straight-line code: the waits are
  // exact counts)
  const __amdgpu_buffer_rsrc_t h0 = buf_rsrc_n(p.h0 + t * nseg * se, (uint32_t)(nseg * se * 4));
  const int64_t lo = n * sd + d;  // the lane's element within a segment's states
  float ds[2][CB], e[2][CB];
  auto load = [&](const int buf, const int64_t s0) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < CB; ++j) {
      const int64_t s = s0 + j < nseg ? s0 + j : nseg - 1;
      ds[buf][j] = dsum[s * sd];
      e[buf][j] = eh[s * se];
    }
  };
  float h = 0.f;
  auto run = [&](const int buf, const int64_t s0) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < CB; ++j) {
      const int64_t s = s0 + j;
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(h), h0, s < nseg ? (int)((s * se + lo) * 4) : 0x7ffffff0, 0, 0);
      const float ld = a * ds[buf][j];
      h = exp2f(fmaxf(ld, -126.0f)) * (h * exp2f(fminf(ld + 126.0f, 0.0f))) + e[buf][j];
    }
  };
  load(0, 0);
  for (int64_t s0 = 0; s0 < nseg; s0 += 2 * CB) {
    load(1, s0 + CB);
    run(0, s0);
    load(0, s0 + 2 * CB);
    run(1, s0 + CB);
  }
}

int cpw_for(int64_t d) { return d % 64 == 0 ? 64 : (d % 32 == 0 ? 32 : 64); }

int64_t pick_seg(int64_t t, int64_t l, int64_t d) {
  // ~4 waves per SIMD over the whole GPU; segments a multiple of the chunk, at least 4 chunks
  const int cpw = cpw_for(d), spw = 64 / cpw;
  const int64_t waves = 16LL * device_cus();
  int64_t nseg = cdiv(waves * spw, t * cdiv(d, cpw));
  if (nseg < 1) nseg = 1;
  int64_t seg = cdiv(cdiv(l, nseg), CH) * CH;
  if (seg < 4 * CH) seg = 4 * CH;
  return seg;
}

}  // namespace

}  // namespace clarus

using namespace clarus;

extern "C" size_t clarus_hip_selective_scan_workspace(int64_t t, int64_t l, int64_t d) {
  if (t <= 0 || l <= 0 || d <= 0) return 0;
  const int64_t nseg = cdiv(l, pick_seg(t, l, d));
  if (nseg == 1) return 16;
  return (size_t)(t * nseg * d * (1 + 2 * NS) * sizeof(float));
}

extern "C" int clarus_hip_selective_scan(const void* u, int32_t u_dtype, const float* dbl, int64_t nc, const float* dt_w,
                                         int64_t r, const float* dt_b, const float* a2, const float* dsk, float* y,
                                         int64_t t, int64_t l, int64_t d, void* scratch, size_t scratch_bytes,
                                         void* stream) {
  clear_error();
  CLARUS_REQUIRE(u && dbl && dt_w && dt_b && a2 && dsk && y && scratch, "selective_scan: null operand");
  CLARUS_REQUIRE(t > 0 && l > 0 && d > 0, "selective_scan: empty problem");
  CLARUS_REQUIRE(u_dtype == DT_BF16 || u_dtype == DT_F32, "selective_scan: u must be bf16 or fp32");
  CLARUS_REQUIRE(r >= 1 && r <= MAXR && nc >= r + 2 * NS, "selective_scan: 1 <= r <= %d and nc >= r + 16", MAXR);
  CLARUS_REQUIRE(t * l * (d > nc ? d : nc) < ((int64_t)1 << 62), "selective_scan: too large");
  const size_t need = clarus_hip_selective_scan_workspace(t, l, d);
  CLARUS_REQUIRE(scratch_bytes >= need, "selective_scan: scratch %zu < %zu bytes", scratch_bytes, need);
  ScanP p{};
  p.u = u; p.dbl = dbl; p.dtw = dt_w; p.dtb = dt_b; p.a2 = a2; p.dsk = dsk; p.y = y;
  p.t = t; p.l = l; p.d = d; p.nc = nc; p.r = (int)r;
  p.seg = pick_seg(t, l, d);
  p.nseg = cdiv(l, p.seg);
  // the carry kernel addresses a chain's start states with 32-bit byte offsets
  CLARUS_REQUIRE(p.nseg * NS * d * (int64_t)sizeof(float) < ((int64_t)1 << 31), "selective_scan: too many segments");
  float* sc = (float*)scratch;
  p.dsum = sc;
  p.eh = sc + t * p.nseg * d;
  p.h0 = p.eh + t * p.nseg * NS * d;
  const int cpw = cpw_for(d), spw = 64 / cpw;
  const dim3 g((unsigned)cdiv(t * p.nseg, spw), (unsigned)cdiv(d, cpw));
  hipStream_t st = (hipStream_t)stream;
  note_kernel("scan_kernel nseg=%lld seg=%lld cpw=%d", (long long)p.nseg, (long long)p.seg, cpw);
#define CLARUS_SCAN(UDT, CPW)                                                                              \
  do {                                                                                                     \
    if (p.nseg > 1) {                                                                                      \
      hipLaunchKernelGGL((scan_kernel<UDT, true, false, CPW>), g, dim3(64), 0, st, p);                     \
      hipLaunchKernelGGL(carry_kernel, dim3((unsigned)cdiv(NS * d, 256), (unsigned)t), dim3(256), 0, st, p); \
      hipLaunchKernelGGL((scan_kernel<UDT, false, true, CPW>), g, dim3(64), 0, st, p);                     \
    } else {                                                                                               \
      hipLaunchKernelGGL((scan_kernel<UDT, false, false, CPW>), g, dim3(64), 0, st, p);                    \
    }                                                                                                      \
  } while (0)
  if (u_dtype == DT_BF16) {
    if (cpw == 32) CLARUS_SCAN(DT_BF16, 32);
    else CLARUS_SCAN(DT_BF16, 64);
  } else {
    if (cpw == 32) CLARUS_SCAN(DT_F32, 32);
    else CLARUS_SCAN(DT_F32, 64);
  }
#undef CLARUS_SCAN
  return check_launch("selective_scan");
}
