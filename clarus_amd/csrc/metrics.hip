// On-device PSNR / SSIM of two uint8 [H, W, 3] images with basicsr's definitions (gfx950):
//   PSNR: 20 log10(peak / sqrt(MSE)), MSE over H W 3 from the exact integer sum of squared
//         differences, peak 1 when max(pred) <= 1 else 255, +inf for identical images.
//   SSIM: basicsr's 3-D SSIM: an 11 x 11 x 11 Gaussian (sigma 1.5, normalised) over (H, W, C)
//         with replicate padding, C1 = (0.01 L)^2, C2 = (0.03 L)^2 (L the same peak), mean of the
//         map over H W 3.
// The 3-D Gaussian is separable: along the length-3 channel axis with replicate padding it is
// the 3 x 3 matrix CM[c][c'] = sum of the taps t with clamp(c + t) = c'; along W and H the
// 11-tap kernel with clamped indices. Moments are accumulated in fp64 (about 128, like the
// reference's fp32 kernels, which they need there against cancellation), so the SSIM mean matches
// the float64 definition to ~1e-12.
//
// Kernels (all sums in a fixed order: deterministic):
//   ssd_max_kernel   per-workgroup int64 sum of squared differences and max(pred) partials
//   ssim_tile_kernel 8 x 32 output pixels x 3 channels per workgroup: the u8 tiles with a
//                    5-pixel clamped halo in LDS, channel mix + horizontal pass into LDS (fp64),
//                    vertical pass and the SSIM map for both constant sets (max(pred) <= 1 or
//                    not, decided later), per-workgroup sums
//   finish_kernel    one workgroup: the partials in order -> res[0] = PSNR, res[1] = SSIM
// replaces python/clarus/metrics.py:59-159 (ssd_max_kernel, ssim_h_kernel, ssim_v_kernel) and
// TritonMetrics.compute (:164-246)
#include <math.h>

#include "capi.hpp"
#include "common.hpp"

namespace clarus {

namespace {

constexpr int SS_BLOCK = 256;
constexpr int SS_PER_THREAD = 64;               // bytes of each image per thread
constexpr int SS_CHUNK = SS_BLOCK * SS_PER_THREAD;  // bytes per workgroup
constexpr int MT_H = 8, MT_W = 32, HALO = 5;
constexpr int MT_RH = MT_H + 2 * HALO, MT_RW = MT_W + 2 * HALO;

struct MetricsP {
  const unsigned char* a;  // pred
  const unsigned char* b;  // gt
  long long* ssd;          // [nb] partial sums of squared differences
  int* mx;                 // [nb] partial max(pred)
  double* ssim;            // [nt][2] partial SSIM sums: constants of peak 1, of peak 255
  double* res;             // [2]
  int64_t h, w, n;         // n = h w 3
  int64_t nb, nt;
};

__global__ void __launch_bounds__(SS_BLOCK) ssd_max_kernel(const MetricsP p) {
  __shared__ long long s_sum[SS_BLOCK];
  __shared__ int s_max[SS_BLOCK];
  const int64_t base = (int64_t)blockIdx.x * SS_CHUNK + (int64_t)threadIdx.x * SS_PER_THREAD;
  long long ssd = 0;
  int mx = 0;
  if (base + SS_PER_THREAD <= p.n && ((uintptr_t)(p.a + base) % 16) == 0 && ((uintptr_t)(p.b + base) % 16) == 0) {
#pragma unroll
    for (int v = 0; v < SS_PER_THREAD / 16; ++v) {
      const u32x4 qa = *reinterpret_cast<const u32x4*>(p.a + base + 16 * v);
      const u32x4 qb = *reinterpret_cast<const u32x4*>(p.b + base + 16 * v);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int x = (qa[i] >> (8 * j)) & 0xff, y = (qb[i] >> (8 * j)) & 0xff;
          ssd += (x - y) * (x - y);
          mx = x > mx ? x : mx;
        }
    }
  } else {
    for (int64_t i = base; i < base + SS_PER_THREAD && i < p.n; ++i) {
      const int x = p.a[i], y = p.b[i];
      ssd += (x - y) * (x - y);
      mx = x > mx ? x : mx;
    }
  }
  s_sum[threadIdx.x] = ssd;
  s_max[threadIdx.x] = mx;
  __syncthreads();
  for (int o = SS_BLOCK / 2; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) {
      s_sum[threadIdx.x] += s_sum[threadIdx.x + o];
      s_max[threadIdx.x] = s_max[threadIdx.x] > s_max[threadIdx.x + o] ? s_max[threadIdx.x] : s_max[threadIdx.x + o];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    p.ssd[blockIdx.x] = s_sum[0];
    p.mx[blockIdx.x] = s_max[0];
  }
}

// the normalised 11-tap Gaussian (sigma 1.5) in fp64, and the channel-mixing matrix
__device__ void gauss_tables(double* g, double* cm) {
  if (threadIdx.x == 0) {
    double s = 0.0;
    for (int i = 0; i < 11; ++i) {
      g[i] = exp(-(double)((i - 5) * (i - 5)) / (2.0 * 1.5 * 1.5));
      s += g[i];
    }
    for (int i = 0; i < 11; ++i) g[i] /= s;
    for (int c = 0; c < 9; ++c) cm[c] = 0.0;
    for (int c = 0; c < 3; ++c)
      for (int t = -5; t <= 5; ++t) {
        int cc = c + t;
        cc = cc < 0 ? 0 : (cc > 2 ? 2 : cc);
        cm[c * 3 + cc] += g[t + 5];
      }
  }
}

__global__ void __launch_bounds__(256) ssim_tile_kernel(const MetricsP p) {
  __shared__ unsigned char ta[MT_RH][MT_RW][3], tb[MT_RH][MT_RW][3];
  __shared__ double hm[5][MT_RH][MT_W][3];  // mixed + horizontally filtered a, b, a^2, b^2, ab
  __shared__ double g[11], cm[9];
  __shared__ double red[2][256];
  const int H = (int)p.h, W = (int)p.w;
  const int tiles_x = (W + MT_W - 1) / MT_W;
  const int ty = blockIdx.x / tiles_x, tx = blockIdx.x - ty * tiles_x;
  const int y0 = ty * MT_H, x0 = tx * MT_W;
  gauss_tables(g, cm);
  // u8 tiles with a clamped (replicate) halo
  for (int e = threadIdx.x; e < MT_RH * MT_RW; e += 256) {
    const int r = e / MT_RW, c = e - r * MT_RW;
    int yy = y0 - HALO + r, xx = x0 - HALO + c;
    yy = yy < 0 ? 0 : (yy > H - 1 ? H - 1 : yy);
    xx = xx < 0 ? 0 : (xx > W - 1 ? W - 1 : xx);
    const int64_t o = ((int64_t)yy * W + xx) * 3;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      ta[r][c][k] = p.a[o + k];
      tb[r][c][k] = p.b[o + k];
    }
  }
  __syncthreads();
  // channel mix + horizontal pass, moments about 128. A thread takes a run of HR consecutive
  // output columns of one (row, channel): it mixes the HR + 10 pixels its windows span once per
  // moment (in registers) and slides the 11 taps over them, instead of mixing every tap's pixel
  // again for each output (11 times the mixing work). Per output the same sums in the same order.
  constexpr int HR = 8, HRUNS = MT_W / HR;
  static_assert(MT_W % HR == 0 && MT_RH * 3 * HRUNS <= 256, "one run per thread");
  if ((int)threadIdx.x < MT_RH * 3 * HRUNS) {
    const int e = threadIdx.x;
    const int r = e / (3 * HRUNS), rem = e - r * (3 * HRUNS), k = rem / HRUNS, c0 = (rem - k * HRUNS) * HR;
    const double w0 = cm[k * 3], w1 = cm[k * 3 + 1], w2 = cm[k * 3 + 2];
#pragma unroll
    for (int q = 0; q < 5; ++q) {
      double m[HR + 10];
#pragma unroll
      for (int j = 0; j < HR + 10; ++j) {
        double mq = 0.0;
#pragma unroll
        for (int kk = 0; kk < 3; ++kk) {
          const double wgt = kk == 0 ? w0 : (kk == 1 ? w1 : w2);
          const double av = (double)ta[r][c0 + j][kk] - 128.0, bv = (double)tb[r][c0 + j][kk] - 128.0;
          if (q == 0) mq += wgt * av;
          else if (q == 1) mq += wgt * bv;
          else if (q == 2) mq += wgt * av * av;
          else if (q == 3) mq += wgt * bv * bv;
          else mq += wgt * av * bv;
        }
        m[j] = mq;
      }
#pragma unroll
      for (int i = 0; i < HR; ++i) {
        double sq = 0.0;
#pragma unroll
        for (int t = 0; t < 11; ++t) sq += g[t] * m[i + t];
        hm[q][r][c0 + i][k] = sq;
      }
    }
  }
  __syncthreads();
  // vertical pass and the SSIM map, both constant sets
  double sum_lo = 0.0, sum_hi = 0.0;
  const double c1l = 0.01 * 0.01, c2l = 0.03 * 0.03, c1h = (0.01 * 255) * (0.01 * 255), c2h = (0.03 * 255) * (0.03 * 255);
  for (int e = threadIdx.x; e < MT_H * MT_W * 3; e += 256) {
    const int r = e / (MT_W * 3), rem = e - r * (MT_W * 3), c = rem / 3, k = rem - (rem / 3) * 3;
    if (y0 + r >= H || x0 + c >= W) continue;
    double v[5] = {0.0, 0.0, 0.0, 0.0, 0.0};
    for (int t = 0; t < 11; ++t)
#pragma unroll
      for (int q = 0; q < 5; ++q) v[q] += g[t] * hm[q][r + t][c][k];
    const double s11 = v[2] - v[0] * v[0], s22 = v[3] - v[1] * v[1], s12 = v[4] - v[0] * v[1];
    const double mu1 = v[0] + 128.0, mu2 = v[1] + 128.0;
    const double m12 = mu1 * mu2, msq = mu1 * mu1 + mu2 * mu2;
    sum_lo += ((2.0 * m12 + c1l) * (2.0 * s12 + c2l)) / ((msq + c1l) * (s11 + s22 + c2l));
    sum_hi += ((2.0 * m12 + c1h) * (2.0 * s12 + c2h)) / ((msq + c1h) * (s11 + s22 + c2h));
  }
  red[0][threadIdx.x] = sum_lo;
  red[1][threadIdx.x] = sum_hi;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) {
      red[0][threadIdx.x] += red[0][threadIdx.x + o];
      red[1][threadIdx.x] += red[1][threadIdx.x + o];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    p.ssim[2 * blockIdx.x] = red[0][0];
    p.ssim[2 * blockIdx.x + 1] = red[1][0];
  }
}

__global__ void __launch_bounds__(256) finish_kernel(const MetricsP p) {
  __shared__ long long s_sum[256];
  __shared__ int s_max[256];
  __shared__ double s_ss[2][256];
  long long ssd = 0;
  int mx = 0;
  for (int64_t i = threadIdx.x; i < p.nb; i += 256) {
    ssd += p.ssd[i];
    mx = p.mx[i] > mx ? p.mx[i] : mx;
  }
  double lo = 0.0, hi = 0.0;
  for (int64_t i = threadIdx.x; i < p.nt; i += 256) {
    lo += p.ssim[2 * i];
    hi += p.ssim[2 * i + 1];
  }
  s_sum[threadIdx.x] = ssd;
  s_max[threadIdx.x] = mx;
  s_ss[0][threadIdx.x] = lo;
  s_ss[1][threadIdx.x] = hi;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) {
      s_sum[threadIdx.x] += s_sum[threadIdx.x + o];
      s_max[threadIdx.x] = s_max[threadIdx.x] > s_max[threadIdx.x + o] ? s_max[threadIdx.x] : s_max[threadIdx.x + o];
      s_ss[0][threadIdx.x] += s_ss[0][threadIdx.x + o];
      s_ss[1][threadIdx.x] += s_ss[1][threadIdx.x + o];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const bool small = s_max[0] <= 1;
    const double mse = (double)s_sum[0] / (double)p.n;
    const double peak = small ? 1.0 : 255.0;
    p.res[0] = mse == 0.0 ? INFINITY : 20.0 * log10(peak / sqrt(mse));
    p.res[1] = (small ? s_ss[0][0] : s_ss[1][0]) / (double)p.n;
  }
}

void metrics_layout(int64_t h, int64_t w, int64_t& nb, int64_t& nt) {
  nb = cdiv(h * w * 3, SS_CHUNK);
  nt = cdiv(h, MT_H) * cdiv(w, MT_W);
}

}  // namespace

}  // namespace clarus

using namespace clarus;

extern "C" size_t clarus_hip_psnr_ssim_workspace(int64_t h, int64_t w) {
  if (h <= 0 || w <= 0) return 0;
  int64_t nb, nt;
  metrics_layout(h, w, nb, nt);
  return (size_t)(nb * 8 + nb * 4 + 16 + nt * 16 + 16);
}

extern "C" int clarus_hip_psnr_ssim(const void* pred, const void* gt, int64_t h, int64_t w, double* res, void* scratch,
                                    size_t scratch_bytes, void* stream) {
  clear_error();
  CLARUS_REQUIRE(pred && gt && res && scratch, "psnr_ssim: null operand");
  CLARUS_REQUIRE(h > 0 && w > 0 && h * w < ((int64_t)1 << 31), "psnr_ssim: bad image size %lld x %lld", (long long)h,
                 (long long)w);
  const size_t need = clarus_hip_psnr_ssim_workspace(h, w);
  CLARUS_REQUIRE(scratch_bytes >= need && aligned(scratch, 16) && aligned(res, 8),
                 "psnr_ssim: scratch %zu < %zu bytes or misaligned", scratch_bytes, need);
  MetricsP p{};
  p.a = (const unsigned char*)pred;
  p.b = (const unsigned char*)gt;
  p.h = h; p.w = w; p.n = h * w * 3;
  metrics_layout(h, w, p.nb, p.nt);
  unsigned char* s = (unsigned char*)scratch;
  p.ssd = (long long*)s;
  p.mx = (int*)(s + p.nb * 8);
  p.ssim = (double*)(s + cdiv(p.nb * 12, 16) * 16);
  p.res = res;
  hipStream_t st = (hipStream_t)stream;
  note_kernel("ssd_max_kernel + ssim_tile_kernel + finish_kernel");
  hipLaunchKernelGGL(ssd_max_kernel, dim3((unsigned)p.nb), dim3(SS_BLOCK), 0, st, p);
  hipLaunchKernelGGL(ssim_tile_kernel, dim3((unsigned)p.nt), dim3(256), 0, st, p);
  hipLaunchKernelGGL(finish_kernel, dim3(1), dim3(256), 0, st, p);
  return check_launch("psnr_ssim");
}
