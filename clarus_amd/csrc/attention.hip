// Restormer MDTA attention map on gfx950:
//   A[n, hd] = softmax( (q / |q|) (k / |k|)^T * t[hd] ),  q, k: [HW, c_h] head slices of qkv.
//
// Stage 1 (gram_partial_kernel), grid (nsplit, batch * heads): each workgroup reduces a
// contiguous pixel range in chunks of 128 pixels. A thread owns one unit of every chunk: 8
// consecutive pixels x one 16-byte channel group of q or k. It loads them one chunk AHEAD into
// registers (two units for fp32), accumulates their squares (the norms, fp32 VALU), transposes the block in
// registers and writes 8 rows of 16 bytes into the LDS tile [channel][pixel] (no bank
// conflicts). Each wave then contracts its 32 pixels with MFMA: the cross blocks Q^T K (NB x NB
// blocks of 16 x 16). bf16 inputs use one bf16 MFMA per block (products exact in fp32); fp32
// inputs are split into bf16 hi + lo and use three (hi hi + hi lo + lo hi, error <= 2^-16
// relative per product). The 4 waves' partials are summed in LDS (the tile's memory, reused)
// in a fixed order and written to scratch as one record per split.
// Stage 2 (gram_reduce_kernel): RS slices of the splits summed per element, in split order.
// Stage 3 (gram_finish_kernel), one workgroup per (image, head): sums the RS slices in order,
// scales by rsqrt(max(|.|^2, 1e-24)) and the temperature, and applies a row softmax.
// The result is deterministic (fixed summation order for a given shape).
#include <mutex>

#include "capi.hpp"
#include "common.hpp"

namespace clarus {

constexpr int GP_CHUNK = 128;  // pixels per chunk (32 per wave)
constexpr int GP_RS = 16;      // reduce slices

// partial record per (image*head, split): [NB*16][NB*16] cross, [NB*16] |q|^2, [NB*16] |k|^2
__host__ __device__ inline int64_t gram_rec_floats(int nb) {
  const int cp = nb * 16;
  return (int64_t)cp * cp + 2 * cp;
}

// LDS of the partial kernel: the transposed chunk [2 CP rows][GP_CHUNK pixels] (+16 B per row),
// reused after the pixel loop as the 4-wave reduction buffer
template <int NB, int DT>
__host__ __device__ constexpr int gram_lds_bytes() {
  return (2 * NB * 16 * (GP_CHUNK * (DT == DT_BF16 ? 2 : 4) + 16)) > (4 * (NB * 16 * NB * 16 + 2 * NB * 16) * 4)
             ? (2 * NB * 16 * (GP_CHUNK * (DT == DT_BF16 ? 2 : 4) + 16))
             : (4 * (NB * 16 * NB * 16 + 2 * NB * 16) * 4);
}

// 8 x 8 transpose of bf16: in[i] = 8 channels of pixel i (u32 pairs), out[c] = 8 pixels of channel c
__device__ __forceinline__ void transpose8x8_bf16(const u32x4 (&in)[8], u32x4 (&out)[8]) {
#pragma unroll
  for (int c = 0; c < 8; ++c) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // out[c] pixels 2j, 2j + 1: channel c of in[2j] and in[2j + 1]
      const unsigned a = in[2 * j][c >> 1], b = in[2 * j + 1][c >> 1];
      out[c][j] = (c & 1) ? __builtin_amdgcn_perm(b, a, 0x07060302u) : __builtin_amdgcn_perm(b, a, 0x05040100u);
    }
  }
}

template <int NB, int DT>
__global__ void __launch_bounds__(256) gram_partial_kernel(const void* __restrict__ qkv, float* __restrict__ part,
                                                           int64_t hw, int c, int ch, int heads,
                                                           int64_t split_len, int nsplit) {
  constexpr int CP = NB * 16;                      // padded head channels
  constexpr int ES = (DT == DT_BF16) ? 2 : 4;
  constexpr int CG = (DT == DT_BF16) ? 8 : 4;      // channels per 16-byte load
  constexpr int TROWB = GP_CHUNK * ES + 16;        // LDS row bytes (+16 B pad)
  constexpr int REC = CP * CP + 2 * CP;
  constexpr int OCT = GP_CHUNK / 8;                // 8-pixel octets per chunk
  __shared__ __attribute__((aligned(16))) unsigned char smem[gram_lds_bytes<NB, DT>()];
  unsigned char* tl = smem;                        // rows [0, CP) q, [CP, 2 CP) k
  float* red = reinterpret_cast<float*>(smem);     // reused after the pixel loop

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lc = lane & 15, lg = lane >> 4;
  const int nh = blockIdx.y;
  const int img = nh / heads, hd = nh - img * heads;
  const int64_t p_begin = (int64_t)blockIdx.x * split_len;
  int64_t p_end = p_begin + split_len;
  if (p_end > hw) p_end = hw;
  const int64_t row_stride = 3LL * c;  // elements per pixel
  const unsigned char* base = (const unsigned char*)qkv + (int64_t)img * hw * row_stride * ES;
  const int groups = ch / CG;          // load groups per head slice
  // units of a chunk: u = tid + 256 t = (which, group) * OCT + octet, octets in consecutive
  // lanes; 2 * groups * OCT <= 256 * UPT (head width <= 64)
  constexpr int UPT = (DT == DT_BF16) ? 1 : 2;
  int octet[UPT], row0[UPT];
  bool active[UPT];
  int64_t coff[UPT];
#pragma unroll
  for (int t = 0; t < UPT; ++t) {
    const int u = tid + 256 * t;
    octet[t] = u % OCT;
    const int wg_ = u / OCT;
    active[t] = wg_ < 2 * groups;
    const int which = active[t] ? wg_ / groups : 0;
    const int grp = active[t] ? wg_ - which * groups : 0;
    coff[t] = (which ? c : 0) + hd * ch + grp * CG;  // channel offset of the unit
    row0[t] = which * CP + grp * CG;                // its first LDS row
  }

  // zero the padded channel rows once (never written by the units)
  for (int u = tid; u < 2 * (CP - ch) * (TROWB / 16); u += 256) {
    const int r = u / (TROWB / 16), col = u - r * (TROWB / 16);
    const int wh = r / (CP - ch), rr = r - wh * (CP - ch);
    *reinterpret_cast<u32x4*>(tl + (wh * CP + ch + rr) * TROWB + col * 16) = u32x4{0u, 0u, 0u, 0u};
  }

  f32x4 cross[NB][NB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) cross[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float sq[UPT][CG];  // sums of squares of each unit's channels (the norms)
#pragma unroll
  for (int t = 0; t < UPT; ++t)
#pragma unroll
    for (int i = 0; i < CG; ++i) sq[t][i] = 0.f;

  u32x4 rq[UPT][8];
  auto fetch = [&](int64_t p0) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < UPT; ++t)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int64_t p = p0 + octet[t] * 8 + i;
        rq[t][i] = (active[t] && p < p_end)
                       ? *reinterpret_cast<const u32x4*>(base + (p * row_stride + coff[t]) * ES)
                       : u32x4{0u, 0u, 0u, 0u};
      }
  };
  auto store_t = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < UPT; ++t) {
      if (!active[t]) continue;
      if constexpr (DT == DT_BF16) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float lo = __uint_as_float(rq[t][i][j] << 16), hi = __uint_as_float(rq[t][i][j] & 0xffff0000u);
            sq[t][2 * j] += lo * lo;
            sq[t][2 * j + 1] += hi * hi;
          }
        u32x4 tr[8];
        transpose8x8_bf16(rq[t], tr);
#pragma unroll
        for (int cc = 0; cc < 8; ++cc)
          *reinterpret_cast<u32x4*>(tl + (row0[t] + cc) * TROWB + octet[t] * 16) = tr[cc];
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float v = __uint_as_float(rq[t][i][j]);
            sq[t][j] += v * v;
          }
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
          unsigned char* d = tl + (row0[t] + cc) * TROWB + octet[t] * 32;
          *reinterpret_cast<u32x4*>(d) = u32x4{rq[t][0][cc], rq[t][1][cc], rq[t][2][cc], rq[t][3][cc]};
          *reinterpret_cast<u32x4*>(d + 16) = u32x4{rq[t][4][cc], rq[t][5][cc], rq[t][6][cc], rq[t][7][cc]};
        }
      }
    }
  };

  if (p_begin < p_end) fetch(p_begin);
  for (int64_t p0 = p_begin; p0 < p_end; p0 += GP_CHUNK) {
    __syncthreads();  // previous chunk's MFMA reads are done
    store_t();
    __syncthreads();
    if (p0 + GP_CHUNK < p_end) fetch(p0 + GP_CHUNK);  // next chunk streams in during the products
    // ---- this wave's 32 pixels: k = wave * 32 + 8 lg + s
    const int kcol = wave * 32 + lg * 8;
    if constexpr (DT == DT_BF16) {
      bf16x8 qf[NB], kf[NB];
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        qf[i] = *reinterpret_cast<const bf16x8*>(tl + (i * 16 + lc) * TROWB + kcol * 2);
        kf[i] = *reinterpret_cast<const bf16x8*>(tl + (CP + i * 16 + lc) * TROWB + kcol * 2);
      }
#pragma unroll
      for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) cross[i][j] = mfma_bf16(qf[i], kf[j], cross[i][j]);
    } else {  // fp32: q = qh + ql, k = kh + kl (bf16), cross = qh kh + qh kl + ql kh
      bf16x8 qh[NB], ql[NB], kh[NB], kl[NB];
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const unsigned char* ra = tl + (i * 16 + lc) * TROWB + kcol * 4;
        const unsigned char* rb = tl + (CP + i * 16 + lc) * TROWB + kcol * 4;
        const f32x4 a0 = *reinterpret_cast<const f32x4*>(ra), a1 = *reinterpret_cast<const f32x4*>(ra + 16);
        const f32x4 b0 = *reinterpret_cast<const f32x4*>(rb), b1 = *reinterpret_cast<const f32x4*>(rb + 16);
        f32x8 qa, ka;
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
          qa.v[s2] = a0[s2]; qa.v[4 + s2] = a1[s2];
          ka.v[s2] = b0[s2]; ka.v[4 + s2] = b1[s2];
        }
        split_bf16(qa, qh[i], ql[i]);
        split_bf16(ka, kh[i], kl[i]);
      }
#pragma unroll
      for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          cross[i][j] = mfma_bf16(qh[i], kh[j], cross[i][j]);
          cross[i][j] = mfma_bf16(qh[i], kl[j], cross[i][j]);
          cross[i][j] = mfma_bf16(ql[i], kh[j], cross[i][j]);
        }
    }
  }

  // ---- reduce the 4 waves (fixed order) and write this split's record
  // D layout: lane holds rows 4 lg + r (q channel within block i), column lc (k channel)
  __syncthreads();  // the transpose tile is free: reuse it as the reduction buffer
  float* my = red + wave * REC;
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int j = 0; j < NB; ++j) my[(i * 16 + lg * 4 + r) * CP + j * 16 + lc] = cross[i][j][r];
  // norms: the OCT threads of a (which, group) unit sum their squares in lane order (the
  // octets of one unit sit in consecutive lanes of one wave)
  if (wave == 0) {
    for (int e = lane; e < 2 * CP; e += 64) my[CP * CP + e] = 0.f;
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < UPT; ++t) {
#pragma unroll
    for (int i = 0; i < CG; ++i) {
      float v = sq[t][i];
#pragma unroll
      for (int o = OCT / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
      if (active[t] && octet[t] == 0) red[CP * CP + row0[t] + i] = v;  // wave 0's record holds the norms
    }
  }
  __syncthreads();
  float* out = part + ((int64_t)nh * nsplit + blockIdx.x) * REC;
  for (int e = tid; e < REC; e += 256)
    out[e] = e < CP * CP ? ((red[e] + red[REC + e]) + red[2 * REC + e]) + red[3 * REC + e] : red[e];
}

// part [nh][nsplit][rec] -> part2 [nh][RS][rec]: slice s sums splits [s * per, (s + 1) * per)
__global__ void __launch_bounds__(256) gram_reduce_kernel(const float* __restrict__ part, float* __restrict__ part2,
                                                          int64_t rec, int nsplit) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int nh = blockIdx.y, sl = blockIdx.z;
  if (e >= rec) return;
  const int per = (nsplit + GP_RS - 1) / GP_RS;
  const int s0 = sl * per;
  const int s1 = s0 + per < nsplit ? s0 + per : nsplit;
  const float* src = part + ((int64_t)nh * nsplit) * rec + e;
  float s = 0.f;
#pragma unroll 8
  for (int sp = s0; sp < s1; ++sp) s += src[(int64_t)sp * rec];
  part2[((int64_t)nh * GP_RS + sl) * rec + e] = s;
}

template <int NB>
__global__ void __launch_bounds__(256) gram_finish_kernel(const float* __restrict__ part2, const float* __restrict__ temp,
                                                          float* __restrict__ out, int ch, int heads) {
  constexpr int CP = NB * 16;
  constexpr int REC = CP * CP + 2 * CP;
  static_assert(REC % 4 == 0, "record of whole 16-byte groups");
  constexpr int PER = (REC / 4 + 255) / 256;  // 16-byte groups per thread
  __shared__ __attribute__((aligned(16))) float g[CP * CP + 2 * CP];  // cross, then |q|^2, |k|^2
  __shared__ float nq[CP], nk[CP];
  const int nh = blockIdx.x;
  const int hd = nh % heads;
  const float* src = part2 + (int64_t)nh * GP_RS * REC;
  // every slice load is issued before any sum is used: one memory latency, 16-byte loads
  f32x4 v[PER][GP_RS];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e4 = threadIdx.x + 256 * i;
#pragma unroll
    for (int sl = 0; sl < GP_RS; ++sl)
      v[i][sl] = e4 < REC / 4 ? *reinterpret_cast<const f32x4*>(src + sl * REC + e4 * 4) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e4 = threadIdx.x + 256 * i;
    f32x4 s4 = v[i][0];
#pragma unroll
    for (int sl = 1; sl < GP_RS; ++sl) s4 += v[i][sl];
    if (e4 < REC / 4) *reinterpret_cast<f32x4*>(g + e4 * 4) = s4;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 2 * CP; e += 256) {
    const float sq = g[CP * CP + e];
    if (e < CP) nq[e] = rsqrtf(fmaxf(sq, 1e-24f));
    else nk[e - CP] = rsqrtf(fmaxf(sq, 1e-24f));
  }
  __syncthreads();
  const float t = temp[hd];
  // four threads per row, CP / 4 columns each (interleaved: column 4 m + q of thread q); max
  // and sum over the four lanes with two butterfly steps
  constexpr int CPT = CP / 4;
  const int i = threadIdx.x >> 2, q = threadIdx.x & 3;
  if (i < CP) {
    float v[CPT];
    float mx = -INFINITY;
    const float si = nq[i] * t;
#pragma unroll
    for (int m = 0; m < CPT; ++m) {
      const int j = 4 * m + q;
      v[m] = (i < ch && j < ch) ? g[i * CP + j] * si * nk[j] : -INFINITY;
      mx = fmaxf(mx, v[m]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
    float sum = 0.f;
#pragma unroll
    for (int m = 0; m < CPT; ++m) {
      v[m] = (4 * m + q < ch) ? expf(v[m] - mx) : 0.f;
      sum += v[m];
    }
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    if (i < ch) {
      const float inv = 1.0f / sum;
      float* o = out + ((int64_t)nh * ch + i) * ch;
#pragma unroll
      for (int m = 0; m < CPT; ++m)
        if (4 * m + q < ch) o[4 * m + q] = v[m] * inv;
    }
  }
}

static int pick_nb(int64_t ch) { return (int)((ch + 15) / 16); }

static int64_t split_len_for(int64_t batch, int64_t heads, int64_t hw) {
  // ~2 workgroups per CU in total, whole chunks per split: long splits amortise the per-split
  // reduction epilogue
  const int64_t wgs = 2LL * device_cus();
  int64_t want = (wgs + batch * heads - 1) / (batch * heads);
  if (want < 1) want = 1;
  int64_t len = (hw + want - 1) / want;
  len = (len + GP_CHUNK - 1) / GP_CHUNK * GP_CHUNK;
  return len < GP_CHUNK ? GP_CHUNK : len;
}

// Launches the three stages with `scratch` as the partials (already checked to be large enough).
static int launch_channel_attention(const void* qkv, int32_t qkv_dtype, const float* temperature, float* out,
                                    int64_t batch, int64_t hw, int64_t c, int64_t heads, void* scratch,
                                    hipStream_t s) {
  const int64_t ch = c / heads;
  const int64_t len = split_len_for(batch, heads, hw);
  const int nsplit = (int)cdiv(hw, len);
  const int nb = pick_nb(ch);
  const int64_t rec = gram_rec_floats(nb);
  dim3 g1((unsigned)nsplit, (unsigned)(batch * heads));
  dim3 g2((unsigned)cdiv(rec, 256), (unsigned)(batch * heads), GP_RS);
  float* part = (float*)scratch;
  float* part2 = part + batch * heads * nsplit * rec;
#define CLARUS_GRAM(NB)                                                                                       \
  do {                                                                                                        \
    if (qkv_dtype == DT_BF16)                                                                                 \
      hipLaunchKernelGGL((gram_partial_kernel<NB, DT_BF16>), g1, dim3(256), 0, s, qkv, part, hw, (int)c,      \
                         (int)ch, (int)heads, len, nsplit);                                                   \
    else                                                                                                      \
      hipLaunchKernelGGL((gram_partial_kernel<NB, DT_F32>), g1, dim3(256), 0, s, qkv, part, hw, (int)c,       \
                         (int)ch, (int)heads, len, nsplit);                                                   \
    hipLaunchKernelGGL(gram_reduce_kernel, g2, dim3(256), 0, s, part, part2, rec, nsplit);                     \
    hipLaunchKernelGGL((gram_finish_kernel<NB>), dim3((unsigned)(batch * heads)), dim3(256), 0, s, part2,     \
                       temperature, out, (int)ch, (int)heads);                                                \
  } while (0)
  note_kernel("gram_partial_kernel + gram_reduce_kernel + gram_finish_kernel nb=%d", nb);
  switch (nb) {
    case 1: CLARUS_GRAM(1); break;
    case 2: CLARUS_GRAM(2); break;
    case 3: CLARUS_GRAM(3); break;
    default: CLARUS_GRAM(4); break;
  }
#undef CLARUS_GRAM
  return check_launch("channel_attention");
}

static int check_channel_attention(const void* qkv, int32_t qkv_dtype, const float* temperature, const float* out,
                                   int64_t batch, int64_t hw, int64_t c, int64_t heads) {
  CLARUS_REQUIRE(qkv && temperature && out, "channel_attention: null operand");
  CLARUS_REQUIRE(batch > 0 && hw > 0 && c > 0 && heads > 0 && c % heads == 0, "channel_attention: bad sizes");
  CLARUS_REQUIRE(qkv_dtype == DT_BF16 || qkv_dtype == DT_F32, "channel_attention: bad dtype");
  const int64_t ch = c / heads;
  CLARUS_REQUIRE(ch % 8 == 0 && ch <= 64, "channel_attention: head width %lld must be a multiple of 8, <= 64",
                 (long long)ch);
  CLARUS_REQUIRE(aligned(qkv, 16) && (c * (qkv_dtype == DT_BF16 ? 2 : 4)) % 16 == 0,
                 "channel_attention: qkv rows must be 16-byte aligned");
  return CLARUS_OK;
}

// The partials of clarus_hip_channel_attention_noalloc: one array per device, resident until the
// process ends. Host code never passes `scratch` itself (in host code the name is only a stand-in
// for the symbol); it uses the device address hipGetSymbolAddress returns, looked up once per
// device with that device current.
constexpr size_t CA_SCRATCH_BYTES = CLARUS_CHANNEL_ATTENTION_SCRATCH_MAX;
__device__ __align__(256) unsigned char scratch[CA_SCRATCH_BYTES];

constexpr int CA_MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[CA_MAX_DEVICES];

// device address of this device's `scratch` (looked up on the first call per device), or null
// with the error text set
static void* device_scratch() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= CA_MAX_DEVICES) {
    set_error("channel_attention_noalloc: no usable current device (%s)", hipGetErrorString(e));
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("channel_attention_noalloc: hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

}  // namespace clarus

using namespace clarus;

extern "C" size_t clarus_hip_channel_attention_workspace(int64_t batch, int64_t hw, int64_t c, int64_t heads) {
  if (batch <= 0 || hw <= 0 || c <= 0 || heads <= 0 || c % heads) return 0;
  const int64_t ch = c / heads;
  const int64_t nsplit = cdiv(hw, split_len_for(batch, heads, hw));
  return (size_t)(batch * heads * (nsplit + GP_RS) * gram_rec_floats(pick_nb(ch)) * sizeof(float));
}

extern "C" int clarus_hip_channel_attention(const void* qkv, int32_t qkv_dtype, const float* temperature, float* out,
                                            int64_t batch, int64_t hw, int64_t c, int64_t heads, void* scratch,
                                            size_t scratch_bytes, void* stream) {
  clear_error();
  int rc = check_channel_attention(qkv, qkv_dtype, temperature, out, batch, hw, c, heads);
  if (rc != CLARUS_OK) return rc;
  CLARUS_REQUIRE(scratch, "channel_attention: null scratch");
  const size_t need = clarus_hip_channel_attention_workspace(batch, hw, c, heads);
  CLARUS_REQUIRE(scratch_bytes >= need, "channel_attention: scratch %zu < %zu bytes", scratch_bytes, need);
  return launch_channel_attention(qkv, qkv_dtype, temperature, out, batch, hw, c, heads, scratch,
                                  (hipStream_t)stream);
}

extern "C" int clarus_hip_channel_attention_noalloc(const void* qkv, int32_t qkv_dtype, const float* temperature,
                                                    float* out, int64_t batch, int64_t hw, int64_t c, int64_t heads,
                                                    void* stream) {
  clear_error();
  int rc = check_channel_attention(qkv, qkv_dtype, temperature, out, batch, hw, c, heads);
  if (rc != CLARUS_OK) return rc;
  const size_t need = clarus_hip_channel_attention_workspace(batch, hw, c, heads);
  CLARUS_REQUIRE(need <= CA_SCRATCH_BYTES,
                 "channel_attention_noalloc: this shape needs %zu bytes of partials, more than the %zu-byte "
                 "static scratch; use clarus_hip_channel_attention with a workspace", need, CA_SCRATCH_BYTES);
  void* ptr = device_scratch();
  if (ptr == nullptr) return CLARUS_ELAUNCH;
  return launch_channel_attention(qkv, qkv_dtype, temperature, out, batch, hw, c, heads, ptr, (hipStream_t)stream);
}
