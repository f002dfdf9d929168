// Mamba selective scan of EVSSM (one direction, no z gate, d_state 8) on gfx950.
//
// For crop t, channel d and state n along the raster sequence l = 0 .. L - 1:
//   delta_l = softplus(dt_raw_l . dt_w[d] + dt_bias[d])
//   h_l[n]  = 2^(delta_l a2[d, n]) h_{l-1}[n] + delta_l B_l[n] u_l[d]      (a2 = A log2(e))
//   y_l[d]  = sum_n C_l[n] h_l[n] + D[d] u_l[d]
// with dbl_l = [dt_raw (r) | B (8) | C (8) | ...] fp32 (row stride nc), u bf16 or fp32, y fp32.
//
// One lane per channel, one wave per (crop, segment, 64 channels): the 8 states live in
// registers and every step is a handful of FMAs and 8 exp2; the step's dbl row is the same for
// the whole wave (scalar loads), u and y are 64 consecutive channels (coalesced). The sequence
// is cut into segments so that enough waves run:
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

__device__ __forceinline__ float softplus(float x) { return x <= 20.0f ? log1pf(expf(x)) : x; }

template <int UDT, bool SUMMARY, bool HAS_H0>
__global__ void __launch_bounds__(64) scan_kernel(const ScanP p) {
  const int lane = threadIdx.x;
  const int64_t d = (int64_t)blockIdx.y * 64 + lane;
  const bool dv = d < p.d;
  const int64_t dl = dv ? d : 0;
  const int64_t ts = blockIdx.x;  // crop * nseg + segment
  const int64_t t = ts / p.nseg, s = ts - t * p.nseg;
  const int64_t l0 = s * p.seg;
  const int64_t l1 = l0 + p.seg < p.l ? l0 + p.seg : p.l;
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
  const float* row = p.dbl + (t * p.l + l0) * p.nc;
  constexpr int UES = UDT == DT_BF16 ? 2 : 4;
  const unsigned char* up = (const unsigned char*)p.u + ((t * p.l + l0) * p.d + dl) * UES;
  float* yp = p.y + (t * p.l + l0) * p.d + dl;
  for (int64_t li = l0; li < l1; ++li) {
    const float uv = UDT == DT_BF16 ? bf16_to_f32(*reinterpret_cast<const unsigned short*>(up))
                                    : *reinterpret_cast<const float*>(up);
    float acc = bias;
#pragma unroll
    for (int i = 0; i < MAXR; ++i)
      if (i < p.r) acc += row[i] * w[i];
    const float delta = softplus(acc);
    const float du = delta * uv;
    float yv = dskip * uv;
#pragma unroll
    for (int n = 0; n < NS; ++n) {
      h[n] = exp2f(delta * a[n]) * h[n] + du * row[p.r + n];
      if (!SUMMARY) yv += h[n] * row[p.r + NS + n];
    }
    if (SUMMARY) dsum += delta;
    else if (dv) *yp = yv;
    row += p.nc;
    up += p.d * UES;
    yp += p.d;
  }
  if (SUMMARY && dv) {
    p.dsum[ts * p.d + d] = dsum;
#pragma unroll
    for (int n = 0; n < NS; ++n) p.eh[(ts * NS + n) * p.d + d] = h[n];
  }
}

// one thread per (crop, state, channel): the segments' start states in order
__global__ void __launch_bounds__(256) carry_kernel(const ScanP p) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // n * d + channel
  const int64_t t = blockIdx.y;
  if (i >= NS * p.d) return;
  const int64_t n = i / p.d, d = i - n * p.d;
  const float a = p.a2[d * NS + n];
  float h = 0.f;
  for (int64_t s = 0; s < p.nseg; ++s) {
    const int64_t ts = t * p.nseg + s;
    p.h0[(ts * NS + n) * p.d + d] = h;
    const float ld = a * p.dsum[ts * p.d + d];
    h = exp2f(fmaxf(ld, -126.0f)) * (h * exp2f(fminf(ld + 126.0f, 0.0f))) + p.eh[(ts * NS + n) * p.d + d];
  }
}

int64_t pick_seg(int64_t t, int64_t l, int64_t d) {
  // ~4 waves per SIMD over the whole GPU, segments of at least 64 steps
  const int64_t waves = 16LL * device_cus();
  const int64_t per = t * cdiv(d, 64);
  int64_t nseg = cdiv(waves, per);
  if (nseg < 1) nseg = 1;
  int64_t seg = cdiv(l, nseg);
  if (seg < 64) seg = 64;
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
  float* sc = (float*)scratch;
  p.dsum = sc;
  p.eh = sc + t * p.nseg * d;
  p.h0 = p.eh + t * p.nseg * NS * d;
  const dim3 g((unsigned)(t * p.nseg), (unsigned)cdiv(d, 64));
  hipStream_t st = (hipStream_t)stream;
  note_kernel("scan_kernel nseg=%lld seg=%lld", (long long)p.nseg, (long long)p.seg);
#define CLARUS_SCAN(UDT)                                                                                   \
  do {                                                                                                     \
    if (p.nseg > 1) {                                                                                      \
      hipLaunchKernelGGL((scan_kernel<UDT, true, false>), g, dim3(64), 0, st, p);                          \
      hipLaunchKernelGGL(carry_kernel, dim3((unsigned)cdiv(NS * d, 256), (unsigned)t), dim3(256), 0, st, p); \
      hipLaunchKernelGGL((scan_kernel<UDT, false, true>), g, dim3(64), 0, st, p);                          \
    } else {                                                                                               \
      hipLaunchKernelGGL((scan_kernel<UDT, false, false>), g, dim3(64), 0, st, p);                         \
    }                                                                                                      \
  } while (0)
  if (u_dtype == DT_BF16) CLARUS_SCAN(DT_BF16);
  else CLARUS_SCAN(DT_F32);
#undef CLARUS_SCAN
  return check_launch("selective_scan");
}
