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
// A thread computes 8 consecutive output channels of one pixel: per tap one 16-byte load of
// each input half (bf16) or two (fp32), fp32 FMAs with the tap weights read from LDS, then
// the gate and a 16-byte store. Lanes are channel-group-minor, so a wave reads whole pixel
// rows; the 3x3 neighbourhood is re-read from L1 / L2. The grid is persistent so the tap
// table ([9][C] fp32, copied as 16-byte vectors) is staged once per block.
#include <algorithm>

#include "capi.hpp"
#include "common.hpp"

namespace clarus {

struct DwP {
  const void* x;
  const float* w;   // [9][C_in] fp32 taps, tap = 3 ky + kx
  const float* b;   // [C_in] fp32 or null
  void* out;
  int64_t n, h, w_, cin, cout;  // cout = cin / 2 with a gate
  int dil, gate, act, x_dt, o_dt;
};

template <int XDT, int GATE>
__global__ void __launch_bounds__(256) dwconv3x3_kernel(const DwP p) {
  extern __shared__ __attribute__((aligned(16))) float wsh[];  // [9][cin] taps, then [cin] bias
  const int cin = (int)p.cin;
  {
    const f32x4* src = reinterpret_cast<const f32x4*>(p.w);  // [9][cin], cin % 8 == 0
    for (int i = threadIdx.x; i < 9 * cin / 4; i += 256) reinterpret_cast<f32x4*>(wsh)[i] = src[i];
    for (int i = threadIdx.x; i < cin; i += 256) wsh[9 * cin + i] = p.b ? p.b[i] : 0.f;
  }
  __syncthreads();

  constexpr int XES = (XDT == DT_BF16) ? 2 : 4;
  const int cout = (int)p.cout;
  const int groups = cout / 8;  // output channel groups of 8
  const int H = (int)p.h, W = (int)p.w_, hw = H * W;
  const int total = (int)(p.n * hw) * groups;  // the host checks that this fits 31 bits
  const int half = GATE ? cout : 0;            // channel offset of the second half
  const unsigned char* X = (const unsigned char*)p.x;
  for (int t = blockIdx.x * 256 + threadIdx.x; t < total; t += gridDim.x * 256) {
    const int pix = t / groups;
    const int c0 = (t - pix * groups) * 8;
    const int img = pix / hw;
    const int r = pix - img * hw;
    const int y = r / W, x = r - (r / W) * W;
    float a1[8], a2[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a1[i] = wsh[9 * cin + c0 + i];
      a2[i] = GATE ? wsh[9 * cin + half + c0 + i] : 0.f;
    }
#pragma unroll
    for (int ky = 0; ky < 3; ++ky) {
      const int yy = y + (ky - 1) * p.dil;
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
        const float* wt = wsh + tap * cin + c0;
        const f32x4 w1a = *reinterpret_cast<const f32x4*>(wt), w1b = *reinterpret_cast<const f32x4*>(wt + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a1[i] = fmaf(w1a[i], v1.v[i], a1[i]);
          a1[4 + i] = fmaf(w1b[i], v1.v[4 + i], a1[4 + i]);
        }
        if constexpr (GATE != 0) {
          const f32x4 w2a = *reinterpret_cast<const f32x4*>(wt + half);
          const f32x4 w2b = *reinterpret_cast<const f32x4*>(wt + half + 4);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            a2[i] = fmaf(w2a[i], v2.v[i], a2[i]);
            a2[4 + i] = fmaf(w2b[i], v2.v[4 + i], a2[4 + i]);
          }
        }
      }
    }
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if constexpr (GATE == 1) o[i] = a1[i] * a2[i];
      else if constexpr (GATE == 2) o[i] = gelu_erf(a1[i]) * a2[i];
      else o[i] = p.act == ACT_GELU ? gelu_erf(a1[i]) : a1[i];
    }
    const int64_t oo = (int64_t)pix * cout + c0;
    if (p.o_dt == DT_BF16) {
      u32x4 q;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        q[i] = (unsigned)f32_to_bf16_bits(o[2 * i]) | ((unsigned)f32_to_bf16_bits(o[2 * i + 1]) << 16);
      *reinterpret_cast<u32x4*>((unsigned short*)p.out + oo) = q;
    } else {
      float* op = (float*)p.out + oo;
      *reinterpret_cast<f32x4*>(op) = f32x4{o[0], o[1], o[2], o[3]};
      *reinterpret_cast<f32x4*>(op + 4) = f32x4{o[4], o[5], o[6], o[7]};
    }
  }
}

// ------------------------------------------------------------------- TLC local mean
// out[i, j, c] = (1 / (k1 k2)) sum_{y = i}^{i + k1 - 1} sum_{x = j}^{j + k2 - 1} X[y, x, c],
// i < OH = h - k1 + 1, j < OW = w - k2 + 1 (the valid windows; python/clarus/ops/
// torch_ref.py:133-141 computes the same map from a 2-D prefix sum). Separable, two passes
// of sliding-window running sums with fp64 accumulators (exact to the fp32 rounding of the
// intermediate): box_v sums k1 rows into V [n, OH, w, c] fp32, box_h sums k2 columns of V.
// A thread owns 8 channels of one column (box_v) or one output row (box_h) over a segment of
// `seg` outputs; lanes are channel-group-minor so a wave touches contiguous NHWC rows.
struct BoxP {
  const void* x;
  float* v;
  void* out;
  int n, h, w, c, k1, k2, oh, ow, seg_v, seg_h, x_dt, o_dt;
  double area;  // k1 * k2
};

__device__ __forceinline__ void add8(double (&s)[8], const f32x8& a, double sign) {
#pragma unroll
  for (int i = 0; i < 8; ++i) s[i] += sign * (double)a.v[i];
}

template <int XDT>
__global__ void __launch_bounds__(256) box_v_kernel(const BoxP p) {
  constexpr int ES = XDT == DT_BF16 ? 2 : 4;
  const int g8 = p.c >> 3;
  const int nseg = (p.oh + p.seg_v - 1) / p.seg_v;
  const int64_t units = (int64_t)p.n * nseg * p.w * g8;
  const int64_t row = (int64_t)p.w * p.c;  // elements per image row
  for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < units; u += (int64_t)gridDim.x * 256) {
    const int g = (int)(u % g8);
    int64_t r = u / g8;
    const int x = (int)(r % p.w);
    r /= p.w;
    const int sg = (int)(r % nseg);
    const int img = (int)(r / nseg);
    const int i0 = sg * p.seg_v;
    const int i1 = i0 + p.seg_v < p.oh ? i0 + p.seg_v : p.oh;
    const unsigned char* col = (const unsigned char*)p.x + (((int64_t)img * p.h * p.w + x) * p.c + g * 8) * ES;
    float* vout = p.v + (((int64_t)img * p.oh * p.w + x) * p.c + g * 8);
    double s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int y = i0; y < i0 + p.k1 - 1; ++y) add8(s, load8<XDT>(col + y * row * ES), 1.0);
#pragma unroll 4
    for (int i = i0; i < i1; ++i) {
      add8(s, load8<XDT>(col + (int64_t)(i + p.k1 - 1) * row * ES), 1.0);
      float* o = vout + (int64_t)i * row;
      *reinterpret_cast<f32x4*>(o) = f32x4{(float)s[0], (float)s[1], (float)s[2], (float)s[3]};
      *reinterpret_cast<f32x4*>(o + 4) = f32x4{(float)s[4], (float)s[5], (float)s[6], (float)s[7]};
      add8(s, load8<XDT>(col + (int64_t)i * row * ES), -1.0);
    }
  }
}

template <int ODT>
__global__ void __launch_bounds__(256) box_h_kernel(const BoxP p) {
  const int g8 = p.c >> 3;
  const int nseg = (p.ow + p.seg_h - 1) / p.seg_h;
  const int64_t units = (int64_t)p.n * p.oh * nseg * g8;
  for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < units; u += (int64_t)gridDim.x * 256) {
    const int g = (int)(u % g8);
    int64_t r = u / g8;
    const int sg = (int)(r % nseg);
    const int64_t irow = r / nseg;  // img * OH + i
    const int j0 = sg * p.seg_h;
    const int j1 = j0 + p.seg_h < p.ow ? j0 + p.seg_h : p.ow;
    const float* vrow = p.v + (irow * p.w) * p.c + g * 8;
    const int64_t orow = (irow * p.ow) * p.c + g * 8;
    double s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int x = j0; x < j0 + p.k2 - 1; ++x) add8(s, load8<DT_F32>(vrow + (int64_t)x * p.c), 1.0);
#pragma unroll 4
    for (int j = j0; j < j1; ++j) {
      add8(s, load8<DT_F32>(vrow + (int64_t)(j + p.k2 - 1) * p.c), 1.0);
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (float)(s[i] / p.area);
      const int64_t oo = orow + (int64_t)j * p.c;
      if constexpr (ODT == DT_BF16) {
        u32x4 q;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          q[i] = (unsigned)f32_to_bf16_bits(o[2 * i]) | ((unsigned)f32_to_bf16_bits(o[2 * i + 1]) << 16);
        *reinterpret_cast<u32x4*>((unsigned short*)p.out + oo) = q;
      } else {
        float* op = (float*)p.out + oo;
        *reinterpret_cast<f32x4*>(op) = f32x4{o[0], o[1], o[2], o[3]};
        *reinterpret_cast<f32x4*>(op + 4) = f32x4{o[4], o[5], o[6], o[7]};
      }
      add8(s, load8<DT_F32>(vrow + (int64_t)j * p.c), -1.0);
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
  const int64_t oh = h - k1 + 1, ow = w - k2 + 1, g8 = c / 8;
  // segments: enough independent running sums to fill the GPU, not much shorter than the window
  auto seg_for = [](int64_t outs, int64_t streams, int64_t want) {
    int64_t nseg = streams >= want ? 1 : (want + streams - 1) / streams;
    int64_t maxseg = (outs + 15) / 16;
    if (nseg > maxseg) nseg = maxseg;
    if (nseg < 1) nseg = 1;
    return (int)((outs + nseg - 1) / nseg);
  };
  BoxP p{x, (float*)scratch, out, (int)n, (int)h, (int)w, (int)c, (int)k1, (int)k2, (int)oh, (int)ow,
         seg_for(oh, n * w * g8, 32768), seg_for(ow, n * oh * g8, 65536), x_dtype, o_dtype,
         (double)k1 * (double)k2};
  const int64_t uv = n * w * g8 * ((oh + p.seg_v - 1) / p.seg_v);
  const int64_t uh = n * oh * g8 * ((ow + p.seg_h - 1) / p.seg_h);
  hipStream_t s = (hipStream_t)stream;
  const unsigned bv = (unsigned)std::min<int64_t>(cdiv(uv, 256), 8192);
  const unsigned bh = (unsigned)std::min<int64_t>(cdiv(uh, 256), 8192);
  if (x_dtype == DT_BF16) hipLaunchKernelGGL(box_v_kernel<DT_BF16>, dim3(bv), dim3(256), 0, s, p);
  else hipLaunchKernelGGL(box_v_kernel<DT_F32>, dim3(bv), dim3(256), 0, s, p);
  if (o_dtype == DT_BF16) hipLaunchKernelGGL(box_h_kernel<DT_BF16>, dim3(bh), dim3(256), 0, s, p);
  else hipLaunchKernelGGL(box_h_kernel<DT_F32>, dim3(bh), dim3(256), 0, s, p);
  return check_launch("boxmean");
}

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
  CLARUS_REQUIRE(aligned(x, 16) && aligned(out, 16) && aligned(w, 16), "dwconv3x3: 16-byte alignment");
  const size_t lds = (size_t)10 * c * sizeof(float);
  CLARUS_REQUIRE(lds <= 160 * 1024, "dwconv3x3: %lld channels exceed the LDS tap table", (long long)c);
  DwP p{x, w, bias, out, n, h, wd, c, cout, dil, gate, act, x_dtype, o_dtype};
  const int64_t total = n * h * wd * (cout / 8);
  // persistent grid: as many blocks as fit the LDS tap table (at most 8 per CU on 256 CUs)
  int64_t per_cu = (int64_t)(160 * 1024) / (int64_t)(lds + 1024);
  per_cu = per_cu < 1 ? 1 : (per_cu > 8 ? 8 : per_cu);
  int64_t blocks = cdiv(total, 256);
  if (blocks > 256 * per_cu) blocks = 256 * per_cu;
  hipStream_t s = (hipStream_t)stream;
#define DW_LAUNCH(XDT, G)                                                                                  \
  do {                                                                                                     \
    static const bool attr = (hipFuncSetAttribute(reinterpret_cast<const void*>(&dwconv3x3_kernel<XDT, G>), \
                                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024), \
                              true);                                                                       \
    (void)attr;                                                                                            \
    hipLaunchKernelGGL((dwconv3x3_kernel<XDT, G>), dim3((unsigned)blocks), dim3(256), lds, s, p);          \
  } while (0)
  if (x_dtype == DT_BF16) {
    if (gate == 1) DW_LAUNCH(DT_BF16, 1); else if (gate == 2) DW_LAUNCH(DT_BF16, 2); else DW_LAUNCH(DT_BF16, 0);
  } else {
    if (gate == 1) DW_LAUNCH(DT_F32, 1); else if (gate == 2) DW_LAUNCH(DT_F32, 2); else DW_LAUNCH(DT_F32, 0);
  }
#undef DW_LAUNCH
  return check_launch("dwconv3x3");
}
