// Depthwise 3x3 convolution with fused gates on gfx950 (NHWC, HBM-bound streaming kernel).
//
//   y[p, c] = b[c] + sum_{ky, kx} w[c, ky, kx] * x[p + dil * (ky - 1, kx - 1), c]   ('same' zero padding)
//   gate 0: out = act(y)                          (C channels)
//   gate 1: out = y[:, :C/2] * y[:, C/2:]         (SimpleGate)
//   gate 2: out = gelu(y[:, :C/2]) * y[:, C/2:]   (GELU gate, Restormer / FFTformer GDFN)
//   act 1 (gate 0 only): out = gelu(y)
// Semantics of the reference backend's dwconv (python/clarus/ops/torch_ref.py:143-155): fp32
// math, one cast to the output dtype at the end.
//
// A workgroup owns a slice of 64 output channels (the taps and bias of its input channels,
// < 5 KiB, staged in LDS once) and walks pixels 32 at a time, so occupancy does not depend
// on C (a tap table of all C channels per workgroup left one workgroup per CU at C = 2048).
// A thread computes 8 consecutive output channels of one pixel: per tap one 16-byte load of
// each input half (bf16) or two (fp32), fp32 FMAs with the tap weights, then the gate and a
// 16-byte store. The 8 lanes of a pixel read 128 contiguous bytes per input half; the 3x3
// neighbourhood is re-read from L1 / L2.
#include <algorithm>

#include "capi.hpp"
#include "gemm_kernel.hpp"

namespace clarus {

struct DwP {
  const void* x;
  const float* w;   // [9][C_in] fp32 taps, tap = 3 ky + kx
  const float* b;   // [C_in] fp32 or null
  void* out;
  int64_t n, h, w_, cin, cout;  // cout = cin / 2 with a gate
  int dil, gate, act, x_dt, o_dt;
};

constexpr int DW_SLICE = 64;  // output channels per workgroup slice (8 lanes of 8 channels)

template <int XDT, int GATE>
__global__ void __launch_bounds__(256) dwconv3x3_kernel(const DwP p) {
  // taps of the slice's input channels: [9][2][DW_SLICE] fp32 (second half with a gate), bias [2][DW_SLICE]
  __shared__ __attribute__((aligned(16))) float wsh[10][2][DW_SLICE];
  const int cin = (int)p.cin, cout = (int)p.cout;
  const int half = GATE ? cout : 0;  // channel offset of the second input half
  const int nslices = (cout + DW_SLICE - 1) / DW_SLICE;
  const int slice = blockIdx.x % nslices;
  const int cs = slice * DW_SLICE;
  for (int i = threadIdx.x; i < 10 * 2 * DW_SLICE; i += 256) {
    const int tap = i / (2 * DW_SLICE), hh = (i / DW_SLICE) & 1, cc = cs + (i % DW_SLICE);
    const int ci = cc + hh * half;
    float v = 0.f;
    if (cc < cout && (GATE || hh == 0)) v = tap < 9 ? p.w[(int64_t)tap * cin + ci] : (p.b ? p.b[ci] : 0.f);
    wsh[tap][hh][i % DW_SLICE] = v;
  }
  __syncthreads();

  constexpr int XES = (XDT == DT_BF16) ? 2 : 4;
  const int o = threadIdx.x & 7;                    // channel lane of the slice
  const int c0 = cs + o * 8;
  const int H = (int)p.h, W = (int)p.w_, hw = H * W;
  const int npix = (int)p.n * hw;                   // the host checks that this fits 31 bits
  const int pstride = (gridDim.x / nslices) * 32;   // pixels per sweep of the grid
  const unsigned char* X = (const unsigned char*)p.x;
  const float* wb = &wsh[0][0][0] + o * 8;          // tap t, half h at wb + (2 t + h) DW_SLICE
  if (c0 >= cout) return;  // no barrier below
  for (int pix = (blockIdx.x / nslices) * 32 + (threadIdx.x >> 3); pix < npix; pix += pstride) {
    const int img = pix / hw;
    const int r = pix - img * hw;
    const int y = r / W, x = r - (r / W) * W;
    float a1[8], a2[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a1[i] = wb[18 * DW_SLICE + i];
      a2[i] = GATE ? wb[19 * DW_SLICE + i] : 0.f;
    }
#pragma unroll
    for (int ky = 0; ky < 3; ++ky) {
      const int yy = y + (ky - 1) * p.dil;
      asm volatile("" ::: "memory");  // one tap row of loads in flight at a time: 8 waves per SIMD
      if (yy < 0 || yy >= H) continue;
#pragma unroll
      for (int kx = 0; kx < 3; ++kx) {
        const int xx = x + (kx - 1) * p.dil;
        if (xx < 0 || xx >= W) continue;
        const int tap = ky * 3 + kx;
        const unsigned char* src = X + ((int64_t)((img * H + yy) * W + xx) * cin + c0) * XES;
        const f32x8 v1 = load8<XDT>(src);
        f32x8 v2;
        if constexpr (GATE != 0) v2 = load8<XDT>(src + (int64_t)half * XES);
        const float* wt = wb + 2 * tap * DW_SLICE;
        const f32x4 w1a = *reinterpret_cast<const f32x4*>(wt), w1b = *reinterpret_cast<const f32x4*>(wt + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a1[i] = fmaf(w1a[i], v1.v[i], a1[i]);
          a1[4 + i] = fmaf(w1b[i], v1.v[4 + i], a1[4 + i]);
        }
        if constexpr (GATE != 0) {
          const f32x4 w2a = *reinterpret_cast<const f32x4*>(wt + DW_SLICE);
          const f32x4 w2b = *reinterpret_cast<const f32x4*>(wt + DW_SLICE + 4);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            a2[i] = fmaf(w2a[i], v2.v[i], a2[i]);
            a2[4 + i] = fmaf(w2b[i], v2.v[4 + i], a2[4 + i]);
          }
        }
      }
    }
    float out[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if constexpr (GATE == 1) out[i] = a1[i] * a2[i];
      else if constexpr (GATE == 2) out[i] = gelu_erf(a1[i]) * a2[i];
      else out[i] = p.act == ACT_GELU ? gelu_erf(a1[i]) : a1[i];
    }
    const int64_t oo = (int64_t)pix * cout + c0;
    if (p.o_dt == DT_BF16) {
      u32x4 q;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        q[i] = (unsigned)f32_to_bf16_bits(out[2 * i]) | ((unsigned)f32_to_bf16_bits(out[2 * i + 1]) << 16);
      *reinterpret_cast<u32x4*>((unsigned short*)p.out + oo) = q;
    } else {
      float* op = (float*)p.out + oo;
      *reinterpret_cast<f32x4*>(op) = f32x4{out[0], out[1], out[2], out[3]};
      *reinterpret_cast<f32x4*>(op + 4) = f32x4{out[4], out[5], out[6], out[7]};
    }
  }
}

// ------------------------------------------------------------------- TLC local mean
// out[i, j, c] = (1 / (k1 k2)) sum_{y = i}^{i + k1 - 1} sum_{x = j}^{j + k2 - 1} X[y, x, c],
// i < OH = h - k1 + 1, j < OW = w - k2 + 1 (the valid windows; python/clarus/ops/
// torch_ref.py:133-141 computes the same map from a 2-D prefix sum). Separable: a vertical
// pass sums k1 rows into V [n, OH, w, c] fp32, a horizontal pass sums k2 columns of V. Both
// are one 1-D sliding-window pass over "lines" (an (x, c) column of a plane, or a c of a V row):
//
//   W(i) = sum_{j = i}^{i + k - 1} X[j],  W(i + 1) = W(i) + X[i + k] - X[i]   (fp64, exact to the
//   final rounding for ordinary data).
//
// Outputs are cut into blocks of k positions (van Herk / Gil-Werman): the windows starting in
// block b cover only blocks b and b + 1. A workgroup owns one block of one plane for a range
// of lines; its T threads per line each own R = k / T consecutive positions. A thread loads
// its R rows of block b and of block b + 1 (16-byte loads: 8 bf16 or 4 fp32 channels), sums
// them (A_s, B_s), exchanges the sums through LDS, and starts its recurrence at
//   W(b k + s R) = sum_{s' >= s} A_s' + sum_{s' < s} B_s'
// so no thread walks a k - 1 element warm-up and every row is read twice.
struct BoxPass {
  const void* x;
  void* y;
  int64_t L, k, lo;   // axis length, window, outputs (L - k + 1)
  int64_t inner;      // elements per axis step (contiguous), a multiple of the lane width
  int64_t outer;      // planes (each L x inner)
  int64_t y_plane;    // output elements per plane (lo x inner)
  int T, R, QW;       // threads per line block, positions per thread, lane groups per workgroup
  int nblk, nqg;      // output blocks per plane, lane-group ranges per plane
  double scale;       // 1 / (k1 k2) on the final pass, 1 otherwise
};


// channel c of a raw 16-byte load: 8 bf16 or 4 fp32
template <int DT>
__device__ __forceinline__ float raw_elem(const u32x4& q, int c) {
  if constexpr (DT == DT_BF16) {
    const unsigned w = q[c >> 1];
    return __uint_as_float((c & 1) ? (w & 0xffff0000u) : (w << 16));
  } else {
    return __uint_as_float(q[c]);
  }
}

// NB: rows loaded per batch and stream (loads in flight per thread); with NB >= R a thread's
// rows are loaded once and stay in registers through the recurrence
template <int XDT, int YDT, int NB>
__global__ void __launch_bounds__(256) box_pass_kernel(const BoxPass p) {
  constexpr int BOX_BATCH = NB;
  constexpr int E = XDT == DT_BF16 ? 8 : 4;  // channels per 16-byte load
  constexpr int XES = XDT == DT_BF16 ? 2 : 4;
  constexpr int YES = YDT == DT_BF16 ? 2 : 4;
  __shared__ double part[2][256][E];         // A_s, B_s of every thread
  const int tid = threadIdx.x;
  const int qi = tid % p.QW, s = tid / p.QW;
  int64_t wg = blockIdx.x;
  const int qg = (int)(wg % p.nqg);
  wg /= p.nqg;
  const int b = (int)(wg % p.nblk);
  const int64_t plane = wg / p.nblk;
  const int64_t e0 = ((int64_t)qg * p.QW + qi) * E;  // first channel of this lane group
  const bool live = e0 < p.inner;
  const unsigned char* xp = (const unsigned char*)p.x + (plane * p.L * p.inner + e0) * XES;
  const int64_t pitch = p.inner * XES;
  const int64_t r0 = (int64_t)b * p.k + (int64_t)s * p.R;  // first position of the thread
  const int64_t pend = (int64_t)s * p.R + p.R < p.k ? (int64_t)s * p.R + p.R : p.k;
  const int nj = pend > (int64_t)s * p.R ? (int)(pend - (int64_t)s * p.R) : 0;  // positions in the block
  // rows r0 + j of block b and r0 + k + j of block b + 1 (zero past the axis)
  auto load_rows = [&](int j0, u32x4 (&va)[BOX_BATCH], u32x4 (&vb)[BOX_BATCH]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < BOX_BATCH; ++j) {
      const int64_t ra = r0 + j0 + j, rb = ra + p.k;
      va[j] = vb[j] = u32x4{0u, 0u, 0u, 0u};
      if (live && j0 + j < nj && ra < p.L) va[j] = *reinterpret_cast<const u32x4*>(xp + ra * pitch);
      if (live && j0 + j < nj && rb < p.L) vb[j] = *reinterpret_cast<const u32x4*>(xp + rb * pitch);
    }
  };
  double sa[E], sb[E];
#pragma unroll
  for (int c = 0; c < E; ++c) sa[c] = sb[c] = 0.0;
  // rows of the last batch stay in registers; when the thread's positions fit one batch
  // (k <= BOX_BATCH T) the recurrence below reuses them instead of reloading
  u32x4 va[BOX_BATCH], vb[BOX_BATCH];
  for (int j0 = 0; j0 < nj; j0 += BOX_BATCH) {
    load_rows(j0, va, vb);
#pragma unroll
    for (int j = 0; j < BOX_BATCH; ++j)
#pragma unroll
      for (int c = 0; c < E; ++c) {
        sa[c] += (double)raw_elem<XDT>(va[j], c);
        sb[c] += (double)raw_elem<XDT>(vb[j], c);
      }
  }
#pragma unroll
  for (int c = 0; c < E; ++c) {
    part[0][tid][c] = sa[c];
    part[1][tid][c] = sb[c];
  }
  __syncthreads();
  double w[E];
#pragma unroll
  for (int c = 0; c < E; ++c) w[c] = 0.0;
  for (int t = 0; t < p.T; ++t) {
    const double* src = part[t >= s ? 0 : 1][t * p.QW + qi];  // A from sub-range s on, B before it
#pragma unroll
    for (int c = 0; c < E; ++c) w[c] += src[c];
  }
  if (!live) return;
  unsigned char* yp = (unsigned char*)p.y + (plane * p.y_plane + e0) * YES;
  // the recurrence over this thread's positions (more than one batch: rows re-read, L1 / L2 hits)
  for (int j0 = 0; j0 < nj; j0 += BOX_BATCH) {
    if (nj > BOX_BATCH) load_rows(j0, va, vb);
#pragma unroll
    for (int j = 0; j < BOX_BATCH; ++j) {
      const int64_t i = r0 + j0 + j;
      if (j0 + j < nj && i < p.lo) {
        unsigned char* o = yp + i * p.inner * YES;
        if constexpr (YDT == DT_BF16) {
          unsigned q[E / 2];
#pragma unroll
          for (int c = 0; c < E / 2; ++c)
            q[c] = (unsigned)f32_to_bf16_bits((float)(w[2 * c] * p.scale)) |
                   ((unsigned)f32_to_bf16_bits((float)(w[2 * c + 1] * p.scale)) << 16);
          if constexpr (E == 8) *reinterpret_cast<u32x4*>(o) = u32x4{q[0], q[1], q[2], q[3]};
          else *reinterpret_cast<u32x2*>(o) = u32x2{q[0], q[1]};
        } else {
#pragma unroll
          for (int c = 0; c < E; c += 4)
            *reinterpret_cast<f32x4*>(o + c * 4) = f32x4{(float)(w[c] * p.scale), (float)(w[c + 1] * p.scale),
                                                         (float)(w[c + 2] * p.scale), (float)(w[c + 3] * p.scale)};
        }
#pragma unroll
        for (int c = 0; c < E; ++c) w[c] += (double)raw_elem<XDT>(vb[j], c) - (double)raw_elem<XDT>(va[j], c);
      }
    }
  }
}

}  // namespace clarus

using namespace clarus;

extern "C" size_t clarus_hip_boxmean_workspace(int64_t n, int64_t h, int64_t w, int64_t c, int64_t k1, int64_t k2) {
  (void)k2;
  if (n <= 0 || h <= 0 || w <= 0 || c <= 0 || k1 < 1 || k1 > h) return 0;
  return (size_t)(n * (h - k1 + 1) * w * c) * sizeof(float);
}

extern "C" int clarus_hip_boxmean(const void* x, int32_t x_dtype, void* out, int32_t o_dtype, int64_t n, int64_t h,
                                  int64_t w, int64_t c, int64_t k1, int64_t k2, void* scratch, size_t scratch_bytes,
                                  void* stream) {
  clear_error();
  CLARUS_REQUIRE(x && out && scratch, "boxmean: null operand");
  CLARUS_REQUIRE(n > 0 && h > 0 && w > 0 && c > 0, "boxmean: empty problem");
  CLARUS_REQUIRE(k1 >= 1 && k1 <= h && k2 >= 1 && k2 <= w, "boxmean: window %lldx%lld outside the %lldx%lld map",
                 (long long)k1, (long long)k2, (long long)h, (long long)w);
  CLARUS_REQUIRE((x_dtype == DT_BF16 || x_dtype == DT_F32) && (o_dtype == DT_BF16 || o_dtype == DT_F32),
                 "boxmean: bad dtype");
  CLARUS_REQUIRE(c % 8 == 0, "boxmean: channels must be a multiple of 8");
  CLARUS_REQUIRE(aligned(x, 16) && aligned(out, 16) && aligned(scratch, 16), "boxmean: 16-byte alignment");
  CLARUS_REQUIRE(n * h * w * c < ((int64_t)1 << 40) && h < (1 << 30) && w < (1 << 30), "boxmean: problem too large");
  const size_t need = clarus_hip_boxmean_workspace(n, h, w, c, k1, k2);
  CLARUS_REQUIRE(scratch_bytes >= need, "boxmean: scratch holds %zu bytes, needs %zu", scratch_bytes, need);
  const int64_t oh = h - k1 + 1;
  hipStream_t s = (hipStream_t)stream;
  // one 1-D pass over `outer` planes of L x inner elements
  auto pass = [&](const void* src, int sdt, void* dst, int ddt, int64_t L, int64_t k, int64_t inner, int64_t outer,
                  double scale) -> bool {
    BoxPass q{};
    q.x = src;
    q.y = dst;
    q.L = L;
    q.k = k;
    q.lo = L - k + 1;
    q.inner = inner;
    q.outer = outer;
    q.y_plane = q.lo * inner;
    // T threads per line block. A thread reads T partial sums (T x 64 B) in the exchange and
    // ~4 k / T rows of 16 B: the two balance at T ~ sqrt(k). T is raised so no lane group of a
    // workgroup is idle (T >= 256 / lane groups in a row), and doubled once more when the GPU
    // would have fewer than ~128 K threads.
    const int E = sdt == DT_BF16 ? 8 : 4;
    const int64_t groups = cdiv(inner, E);
    const int64_t lines = outer * cdiv(q.lo, k) * groups;
    int T0 = 1;
    while ((int64_t)(2 * T0) * (2 * T0) <= k) T0 *= 2;
    int T = T0;
    while (T < 256 && T * groups < 256) T *= 2;
    if (T == T0 && T < 256 && lines * T < 131072) T *= 2;
    // long windows take more threads while each keeps >= 6 positions (NAFNet-w64 720p, cold, us:
    // level 0, k = 384, 128.7 -> 117.4; level 1, k = 192, 62.5 -> 60.9); at 3 positions per
    // thread (k = 96, 48) the exchange outweighs the rows: 35.1 -> 47.7 and 24.9 -> 35.7
    while (T < 256 && lines * T < 262144 && cdiv(k, (int64_t)(2 * T)) >= 6) T *= 2;
    q.T = T;
    q.R = (int)cdiv(k, T);
    q.QW = 256 / T;
    q.nblk = (int)cdiv(q.lo, k);
    q.nqg = (int)cdiv(cdiv(inner, E), q.QW);
    q.scale = scale;
    const int64_t blocks = outer * q.nblk * q.nqg;
    if (blocks >= ((int64_t)1 << 31)) return false;
    // rows per batch: 8, the rows reloaded for the recurrence when R > 8; all R rows kept in
    // registers (one wave per SIMD) where that measured faster, us: bf16 rows with R = 24 (NAFNet
    // level 0, vertical pass) 64.0 vs 70-74, fp32 rows with R = 12 (level 1, horizontal) 28.3 vs
    // 30.4; not kept: bf16 R = 12 (level 1 vertical) 39.1 vs 30-31, fp32 R = 24 64.1 vs 59.4
    const int nb = (sdt == DT_BF16 && q.R > 16 && q.R <= 24) ? 24 : (sdt == DT_F32 && q.R > 8 && q.R <= 16) ? 16 : 8;
#define CLARUS_BOX_LAUNCH(NB_)                                                                             \
  if (sdt == DT_BF16) hipLaunchKernelGGL((box_pass_kernel<DT_BF16, DT_F32, NB_>), dim3((unsigned)blocks), dim3(256), 0, s, q); \
  else if (ddt == DT_BF16) hipLaunchKernelGGL((box_pass_kernel<DT_F32, DT_BF16, NB_>), dim3((unsigned)blocks), dim3(256), 0, s, q); \
  else hipLaunchKernelGGL((box_pass_kernel<DT_F32, DT_F32, NB_>), dim3((unsigned)blocks), dim3(256), 0, s, q);
    if (nb == 8) { CLARUS_BOX_LAUNCH(8) }
    else if (nb == 16) { CLARUS_BOX_LAUNCH(16) }
    else { CLARUS_BOX_LAUNCH(24) }
#undef CLARUS_BOX_LAUNCH
    return true;
  };
  // vertical: planes are images, lines the (x, c) columns; horizontal: planes are V rows
  CLARUS_REQUIRE(pass(x, x_dtype, scratch, DT_F32, h, k1, w * c, n, 1.0), "boxmean: too many workgroups");
  CLARUS_REQUIRE(pass(scratch, DT_F32, out, o_dtype, w, k2, c, n * oh, 1.0 / ((double)k1 * (double)k2)),
                 "boxmean: too many workgroups");
  return check_launch("boxmean");
}

// Sliding-window variant for dilation 1 and narrow rows. A lane owns 8
// consecutive channels of ONE input half (with a gate, lanes l and l + 32 hold the two halves of
// the same output channels) and walks a run of R consecutive pixels along a row: per step it
// loads one new column of 3 pixels (3 16-byte loads per output instead of 9 per half) and adds
// it to the up to 3 outputs whose window contains that column, so 3 partial outputs are live.
// Its 72 tap weights and 8 biases stay in registers for the whole run. SimpleGate / GELU gate
// combine the halves with a cross-lane exchange (l <-> l ^ 32). The 8 lanes of a pixel read
// 128 contiguous bytes per half; a wave covers 8 (gate: 4) runs of 64 channels.
// Per output the taps are summed column by column (kx outer, ky inner) after the bias.
template <int XDT, int GATE, int R>
__global__ void __launch_bounds__(256) dw_rows_kernel(const DwP p) {
  constexpr int XES = (XDT == DT_BF16) ? 2 : 4;
  constexpr int RPW = GATE ? 4 : 8;  // runs per wave
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hf = GATE ? (lane >> 5) : 0;
  const int l = GATE ? (lane & 31) : lane;
  const int cg = l & 7, rw = l >> 3;
  const int cout = (int)p.cout, cin = (int)p.cin;
  const int nslices = (cout + DW_SLICE - 1) / DW_SLICE;
  const int slice = blockIdx.x % nslices;
  const int c0 = slice * DW_SLICE + cg * 8;      // first output channel of the lane
  const bool active = c0 < cout;                 // the same for both halves of a pair
  const int ci = c0 + (GATE ? hf * cout : 0);    // first input channel of the lane's half
  float wt[9][8], bs[8];
#pragma unroll
  for (int t = 0; t < 9; ++t)
#pragma unroll
    for (int i = 0; i < 8; ++i) wt[t][i] = active ? p.w[(int64_t)t * cin + ci + i] : 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) bs[i] = (active && p.b) ? p.b[ci + i] : 0.f;

  const int H = (int)p.h, W = (int)p.w_;
  const int rpr = (W + R - 1) / R;               // runs per image row
  const int total = (int)p.n * H * rpr;          // the host checks that this fits 31 bits
  const int per_wg = 4 * RPW;
  const int stride = (gridDim.x / nslices) * per_wg;
  const unsigned char* X = (const unsigned char*)p.x;
  for (int run = (blockIdx.x / nslices) * per_wg + wave * RPW + rw; run < total; run += stride) {
    const int img = run / (H * rpr);
    const int rr = run - img * H * rpr;
    const int y = rr / rpr;
    const int x0 = (rr - y * rpr) * R;
    const unsigned char* rowp[3];
    bool rok[3];
#pragma unroll
    for (int ky = 0; ky < 3; ++ky) {
      const int yy = y + ky - 1;
      rok[ky] = active && yy >= 0 && yy < H;
      rowp[ky] = X + ((int64_t)(img * H + (rok[ky] ? yy : 0)) * W * cin + ci) * XES;
    }
    // every load of the run is issued before the first FMA (one memory round trip per run)
    RawFrag<XDT> raw[R + 2][3];
#pragma unroll
    for (int cc = 0; cc < R + 2; ++cc) {
      const int x = x0 - 1 + cc;
      const bool xok = x >= 0 && x < W;
#pragma unroll
      for (int ky = 0; ky < 3; ++ky)
        raw[cc][ky] = (xok && rok[ky]) ? raw_load<XDT>(rowp[ky] + (int64_t)x * cin * XES) : raw_zero<XDT>();
    }
    float acc[3][8];
#pragma unroll
    for (int cc = 0; cc < R + 2; ++cc) {  // column x0 - 1 + cc
      if (cc < R) {
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[cc % 3][i] = bs[i];
      }
      f32x8 col[3];
#pragma unroll
      for (int ky = 0; ky < 3; ++ky) col[ky] = raw_f32<XDT>(raw[cc][ky]);
#pragma unroll
      for (int j = cc - 2; j <= cc; ++j) {  // outputs whose window holds this column (kx = cc - j)
        if (j < 0 || j >= R) continue;
#pragma unroll
        for (int ky = 0; ky < 3; ++ky)
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[j % 3][i] = fmaf(wt[ky * 3 + cc - j][i], col[ky].v[i], acc[j % 3][i]);
      }
      if (cc < 2) continue;
      // output j = cc - 2 is complete
      const int j = cc - 2;
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = acc[j % 3][i];
      if constexpr (GATE != 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float o = __shfl_xor(v[i], 32, 64);  // the other half of the same channel
          v[i] = GATE == 1 ? v[i] * o : gelu_erf(v[i]) * o;
        }
      } else if (p.act == ACT_GELU) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = gelu_erf(v[i]);
      }
      const int xo = x0 + j;
      if (hf != 0 || !active || xo >= W) continue;
      const int64_t oo = ((int64_t)(img * H + y) * W + xo) * cout + c0;
      if (p.o_dt == DT_BF16) {
        u32x4 q;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          q[i] = (unsigned)f32_to_bf16_bits(v[2 * i]) | ((unsigned)f32_to_bf16_bits(v[2 * i + 1]) << 16);
        *reinterpret_cast<u32x4*>((unsigned short*)p.out + oo) = q;
      } else {
        float* op = (float*)p.out + oo;
        *reinterpret_cast<f32x4*>(op) = f32x4{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<f32x4*>(op + 4) = f32x4{v[4], v[5], v[6], v[7]};
      }
    }
  }
}

// LDS-tiled variant for bf16 input with a gate. A workgroup owns a slice of 64 output channels
// and walks tiles of TH x DWT_TW output pixels. The tile's input (its rows and columns plus a
// one-pixel halo, both input halves: (TH + 2) x (DWT_TW + 2) pixels x 256 bytes) is copied
// global -> LDS once by direct copies, pixels outside the image from a zero page, so every input
// vector crosses the vector-memory path once per tile instead of 9 times. With NBUF = 2 the next
// tile's copies go out before the current tile is computed. Lane (run, cq) owns output column
// `run` of the tile and channels 4 cq .. 4 cq + 3 of both halves, keeps their 72 taps and 8
// biases in registers and walks its column down the tile: per input row six 8-byte LDS reads
// (both halves of the pixels left, at and right of the column; the next row's issued before this
// row's FMAs) feed the up to 3 outputs whose window holds that row, and the gate is formed in the
// lane. In LDS a pixel's two 128-byte halves are swapped when its column is odd, so the 4 runs of
// a wave read both bank halves. Per output the sum runs bias, then ky outer, kx inner (the order of
// dwconv3x3_kernel). Stores are buffer stores whose range drops the lanes outside the image, so
// every wave issues the same TH stores per tile and the wait for the next tile's copies can leave
// them in flight.
constexpr int DWT_TW = 16;
template <int TH>
struct DwTile {
  static constexpr int ROWS = TH + 2, COLS = DWT_TW + 2;
  static constexpr int UNITS = ROWS * COLS * 2 * 8;    // 16-byte units: pixel, half, 8 units of 128 B
  static constexpr int COPIES = (UNITS + 255) / 256;   // copies per lane (4 waves of 64 units each)
  static constexpr int BYTES = COPIES * 256 * 16;
};
static __device__ __attribute__((aligned(256))) unsigned char g_dw_zero[256];

template <int GATE, int TH, int NBUF, int ODT>
__global__ void __launch_bounds__(256) dw_tile_kernel(const DwP p) {
  static_assert(GATE == 1 || GATE == 2, "gated form only");
  using G = DwTile<TH>;
  constexpr int OES = ODT == DT_BF16 ? 2 : 4;
  __shared__ __attribute__((aligned(16))) unsigned char tile[NBUF][G::BYTES];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int cq = lane & 15, run = wave * 4 + (lane >> 4);
  const int cout = (int)p.cout, cin = (int)p.cin;
  const int nslices = (cout + DW_SLICE - 1) / DW_SLICE;
  const int slice = blockIdx.x % nslices;
  const int c0 = slice * DW_SLICE + cq * 4;  // first output channel of the lane
  const bool active = c0 < cout;             // cout % 8 == 0: all 4 channels or none
  float wt[2][9][4], bs[2][4];               // [half][tap][channel]
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int ci = c0 + h * cout;
#pragma unroll
    for (int t = 0; t < 9; ++t) {
      const f32x4 a = active ? *reinterpret_cast<const f32x4*>(p.w + (int64_t)t * cin + ci) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 4; ++i) wt[h][t][i] = a[i];
    }
    const f32x4 b = (active && p.b) ? *reinterpret_cast<const f32x4*>(p.b + ci) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) bs[h][i] = b[i];
  }

  const int H = (int)p.h, W = (int)p.w_;
  const int tiles_x = (W + DWT_TW - 1) / DWT_TW, tiles_y = (H + TH - 1) / TH;
  const int ptiles = (int)p.n * tiles_y * tiles_x;  // the host checks that this fits 31 bits
  const int stride = gridDim.x / nslices;
  const unsigned char* X = (const unsigned char*)p.x;
  // the host checks that the output is under 2^31 - 16 bytes: 32-bit buffer offsets
  const __amdgpu_buffer_rsrc_t orc = buf_rsrc_n(p.out, (uint32_t)(p.n * p.h * p.w_ * p.cout * OES));
  // copy j of a lane fills unit u = (wave + 4 j) * 64 + lane of the tile's LDS image: pixel u / 16
  // of the (TH + 2) x (DWT_TW + 2) halo tile, 16 bytes (u % 8) of half ((u / 8) % 2) ^ (column % 2)
  // of the slice's 128
  const int k = lane & 7, slot = (lane >> 3) & 1;
  const bool k_real = slice * DW_SLICE + k * 8 < cout;
  auto tile_pos = [&](int t, int& img, int& y0, int& x0) __attribute__((always_inline)) {
    img = t / (tiles_y * tiles_x);
    const int rem = t - img * tiles_y * tiles_x;
    const int ty = rem / tiles_x;
    y0 = ty * TH;
    x0 = (rem - ty * tiles_x) * DWT_TW;
  };
  auto issue = [&](int t, unsigned char* dst) __attribute__((always_inline)) {
    int img, y0, x0;
    tile_pos(t, img, y0, x0);
#pragma unroll
    for (int j = 0; j < G::COPIES; ++j) {
      const int pix = ((wave + 4 * j) * 64 + lane) >> 4;
      const int r = pix / G::COLS, c = pix - (pix / G::COLS) * G::COLS;
      const int seg = slot ^ (c & 1);
      const int yy = y0 - 1 + r, xx = x0 - 1 + c;
      const bool ok = k_real && pix < G::ROWS * G::COLS && yy >= 0 && yy < H && xx >= 0 && xx < W;
      const int yc = min(max(yy, 0), H - 1), xc = min(max(xx, 0), W - 1);  // an address in the image
      const unsigned char* src =
          ok ? X + (((int64_t)img * H + yc) * W + xc) * cin * 2 + (slice * DW_SLICE + seg * cout + k * 8) * 2 : g_dw_zero;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                       (__attribute__((address_space(3))) void*)(dst + (wave + 4 * j) * 1024), 16, 0, 0);
    }
  };
  // byte offset of half h of tile pixel (row, column) for this lane's channels
  auto lds_at = [&](int row, int col, int h) __attribute__((always_inline)) {
    return (row * G::COLS + col) * 256 + ((h ^ (col & 1)) * 128) + cq * 8;
  };
  int t = blockIdx.x / nslices;
  if (NBUF == 2 && t < ptiles) issue(t, tile[0]);
  for (int it = 0; t < ptiles; ++it, t += stride) {
    unsigned char* cur = tile[NBUF == 2 ? (it & 1) : 0];
    if constexpr (NBUF == 2) {
      // this tile's copies are older than the previous tile's TH stores
      if (it == 0) wait_vmcnt<0>(); else wait_vmcnt<TH>();
      __syncthreads();  // copies landed; every wave is done with the other buffer
      if (t + stride < ptiles) issue(t + stride, tile[(it & 1) ^ 1]);
    } else {
      issue(t, cur);
      wait_vmcnt<0>();
      __syncthreads();
    }
    int img, y0, x0;
    tile_pos(t, img, y0, x0);
    const int xo = x0 + run;
    float acc[3][2][4];
    u32x2 q[2][3][2];  // [row parity][dx][half]: raw bf16 of the row being summed and the next
#pragma unroll
    for (int dx = 0; dx < 3; ++dx)
#pragma unroll
      for (int h = 0; h < 2; ++h) q[0][dx][h] = *reinterpret_cast<const u32x2*>(cur + lds_at(0, run + dx, h));
#pragma unroll
    for (int ir = 0; ir < G::ROWS; ++ir) {  // input row y0 - 1 + ir
      if (ir + 1 < G::ROWS) {
#pragma unroll
        for (int dx = 0; dx < 3; ++dx)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            q[(ir + 1) & 1][dx][h] = *reinterpret_cast<const u32x2*>(cur + lds_at(ir + 1, run + dx, h));
      }
      if (ir < TH) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[ir % 3][h][i] = bs[h][i];
      }
      float v[3][2][4];
#pragma unroll
      for (int dx = 0; dx < 3; ++dx)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const u32x2 r = q[ir & 1][dx][h];
          v[dx][h][0] = __uint_as_float(r[0] << 16);
          v[dx][h][1] = __uint_as_float(r[0] & 0xffff0000u);
          v[dx][h][2] = __uint_as_float(r[1] << 16);
          v[dx][h][3] = __uint_as_float(r[1] & 0xffff0000u);
        }
#pragma unroll
      for (int o = ir - 2; o <= ir; ++o) {  // outputs whose window holds this row (ky = ir - o)
        if (o < 0 || o >= TH) continue;
#pragma unroll
        for (int dx = 0; dx < 3; ++dx)
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              acc[o % 3][h][i] = fmaf(wt[h][(ir - o) * 3 + dx][i], v[dx][h][i], acc[o % 3][h][i]);
      }
      if (ir < 2) continue;
      const int o = ir - 2;  // output row y0 + o is complete
      float g[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = acc[o % 3][0][i], b = acc[o % 3][1][i];
        if constexpr (GATE == 1) g[i] = a * b;
        else g[i] = gelu_erf(a) * b;
      }
      const int yo = y0 + o;
      const bool keep = active && yo < H && xo < W;
      const int oo = keep ? (int)(((((int64_t)img * H + yo) * W + xo) * cout + c0) * OES) : 0x7ffffff0;
      if constexpr (ODT == DT_BF16) {
        u32x2 w2;
        w2[0] = (unsigned)f32_to_bf16_bits(g[0]) | ((unsigned)f32_to_bf16_bits(g[1]) << 16);
        w2[1] = (unsigned)f32_to_bf16_bits(g[2]) | ((unsigned)f32_to_bf16_bits(g[3]) << 16);
        __builtin_amdgcn_raw_buffer_store_b64(w2, orc, oo, 0, 0);
      } else {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, f32x4{g[0], g[1], g[2], g[3]}), orc, oo, 0, 0);
      }
    }
    if constexpr (NBUF == 1) __syncthreads();  // every wave is done with the tile before the next copies land
  }
}

constexpr int DW_RUN = 4;  // pixels per run of dw_rows_kernel

extern "C" int clarus_hip_dwconv3x3(const void* x, int32_t x_dtype, const float* w, const float* bias, void* out,
                                    int32_t o_dtype, int64_t n, int64_t h, int64_t wd, int64_t c, int32_t dil,
                                    int32_t gate, int32_t act, void* stream) {
  clear_error();
  CLARUS_REQUIRE(x && w && out, "dwconv3x3: null operand");
  CLARUS_REQUIRE(n > 0 && h > 0 && wd > 0 && c > 0, "dwconv3x3: empty problem");
  CLARUS_REQUIRE((x_dtype == DT_BF16 || x_dtype == DT_F32) && (o_dtype == DT_BF16 || o_dtype == DT_F32),
                 "dwconv3x3: bad dtype");
  CLARUS_REQUIRE(gate >= 0 && gate <= 2 && (act == 0 || (act == ACT_GELU && gate == 0)) && dil >= 1,
                 "dwconv3x3: bad gate / act / dilation");
  const int64_t cout = gate ? c / 2 : c;
  CLARUS_REQUIRE((gate == 0 || c % 2 == 0) && cout % 8 == 0, "dwconv3x3: output channels must be a multiple of 8");
  CLARUS_REQUIRE(n * h * wd * (cout / 8) < ((int64_t)1 << 31) && n * h * wd * c < ((int64_t)1 << 40),
                 "dwconv3x3: problem too large for 32-bit pixel indexing");
  CLARUS_REQUIRE(aligned(x, 16) && aligned(out, 16), "dwconv3x3: 16-byte alignment");
  DwP p{x, w, bias, out, n, h, wd, c, cout, dil, gate, act, x_dtype, o_dtype};
  // workgroups: channel slices x pixel chunks of 32, persistent with every workgroup resident
  // (a grid-stride loop over more workgroups than fit leaves a tail of late starters)
  const int64_t nslices = cdiv(cout, DW_SLICE);
  const int64_t chunks = cdiv(n * h * wd, 32);
  hipStream_t s = (hipStream_t)stream;
#define DW_LAUNCH(XDT, G)                                                                                       \
  do {                                                                                                          \
    auto fn = &dwconv3x3_kernel<XDT, G>;                                                                        \
    static const int per_cu = [&] {                                                                             \
      int k = 0;                                                                                                \
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&k, reinterpret_cast<const void*>(fn), 256, 0) !=       \
              hipSuccess ||                                                                                     \
          k < 1)                                                                                                \
        k = 1;                                                                                                  \
      return k;                                                                                                 \
    }();                                                                                                        \
    const int64_t cap = std::max<int64_t>(1, (int64_t)device_cus() * per_cu / nslices);                                        \
    const unsigned blocks = (unsigned)(nslices * std::min<int64_t>(chunks, cap));                               \
    hipLaunchKernelGGL(fn, dim3(blocks), dim3(256), 0, s, p);                                                   \
  } while (0)
  // sliding-window kernel for dilation 1 and up to 256 input channels (measured on the NAFNet
  // 720p levels: 127 vs 151 us at 128 channels, even at 256, slower from 512 channels on, where
  // the per-pixel kernel's higher occupancy wins): runs of DW_RUN pixels, workgroups of 16
  // (gate) / 32 runs
  // LDS-tiled kernel: bf16 input with a gate, dilation 1, 16-byte aligned taps and bias, an
  // output under 2^31 - 16 bytes (32-bit buffer offsets). Tiles of 6 rows, two buffers (two
  // workgroups per CU at 225 VGPRs; NAFNet-w64 720p levels 0-4, cold, us: 91 / 50 / 31 / 19 / 14
  // against 128 / 73 / 45 / 28 / 17 for the kernels below; 8-row tiles with one buffer 95 / 51 /
  // 32 / 20 / 13)
  const int64_t o_bytes = n * h * wd * cout * (o_dtype == DT_BF16 ? 2 : 4);
  if (dil == 1 && gate != 0 && x_dtype == DT_BF16 && aligned(w, 16) && (!bias || aligned(bias, 16)) &&
      o_bytes < ((int64_t)1 << 31) - 16) {
    constexpr int TH = 6, NBUF = 2;
    const int64_t ptiles = n * cdiv(h, TH) * cdiv(wd, DWT_TW);
    CLARUS_REQUIRE(ptiles < ((int64_t)1 << 31), "dwconv3x3: problem too large for 32-bit tile indexing");
#define DW_TILE(G, ODT)                                                                                         \
  do {                                                                                                          \
    auto fn = &dw_tile_kernel<G, TH, NBUF, ODT>;                                                                \
    static const int per_cu = [&] {                                                                             \
      int k = 0;                                                                                                \
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&k, reinterpret_cast<const void*>(fn), 256, 0) !=       \
              hipSuccess ||                                                                                     \
          k < 1)                                                                                                \
        k = 1;                                                                                                  \
      return k;                                                                                                 \
    }();                                                                                                        \
    const int64_t cap = std::max<int64_t>(1, (int64_t)device_cus() * per_cu / nslices);                        \
    const unsigned blocks = (unsigned)(nslices * std::min<int64_t>(ptiles, cap));                               \
    hipLaunchKernelGGL(fn, dim3(blocks), dim3(256), 0, s, p);                                                   \
  } while (0)
    note_kernel("dw_tile_kernel gate=%d th=%d nbuf=%d", gate, TH, NBUF);
    if (o_dtype == DT_BF16) {
      if (gate == 1) DW_TILE(1, DT_BF16); else DW_TILE(2, DT_BF16);
    } else {
      if (gate == 1) DW_TILE(1, DT_F32); else DW_TILE(2, DT_F32);
    }
#undef DW_TILE
    return check_launch("dwconv3x3");
  }
  if (dil == 1 && c <= 256) {
    const int64_t runs = n * h * cdiv(wd, DW_RUN);
    CLARUS_REQUIRE(runs < ((int64_t)1 << 31), "dwconv3x3: problem too large for 32-bit run indexing");
    const int64_t rchunks = cdiv(runs, gate ? 16 : 32);
#define DW_ROWS(XDT, G)                                                                                         \
  do {                                                                                                          \
    auto fn = &dw_rows_kernel<XDT, G, DW_RUN>;                                                                  \
    static const int per_cu = [&] {                                                                             \
      int k = 0;                                                                                                \
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&k, reinterpret_cast<const void*>(fn), 256, 0) !=       \
              hipSuccess ||                                                                                     \
          k < 1)                                                                                                \
        k = 1;                                                                                                  \
      return k;                                                                                                 \
    }();                                                                                                        \
    const int64_t cap = std::max<int64_t>(1, (int64_t)device_cus() * per_cu / nslices);                                        \
    const unsigned blocks = (unsigned)(nslices * std::min<int64_t>(rchunks, cap));                              \
    hipLaunchKernelGGL(fn, dim3(blocks), dim3(256), 0, s, p);                                                   \
  } while (0)
    if (x_dtype == DT_BF16) {
      if (gate == 1) DW_ROWS(DT_BF16, 1); else if (gate == 2) DW_ROWS(DT_BF16, 2); else DW_ROWS(DT_BF16, 0);
    } else {
      if (gate == 1) DW_ROWS(DT_F32, 1); else if (gate == 2) DW_ROWS(DT_F32, 2); else DW_ROWS(DT_F32, 0);
    }
#undef DW_ROWS
    return check_launch("dwconv3x3");
  }
  if (x_dtype == DT_BF16) {
    if (gate == 1) DW_LAUNCH(DT_BF16, 1); else if (gate == 2) DW_LAUNCH(DT_BF16, 2); else DW_LAUNCH(DT_BF16, 0);
  } else {
    if (gate == 1) DW_LAUNCH(DT_F32, 1); else if (gate == 2) DW_LAUNCH(DT_F32, 2); else DW_LAUNCH(DT_F32, 0);
  }
#undef DW_LAUNCH
  return check_launch("dwconv3x3");
}
