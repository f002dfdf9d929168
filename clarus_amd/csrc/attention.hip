// Restormer MDTA attention map on gfx950:
//   A[n, hd] = softmax( (q / |q|) (k / |k|)^T * t[hd] ),  q, k: [HW, c_h] head slices of qkv.
//
// Stage 1 (gram_partial_kernel), grid (nsplit, batch * heads): each workgroup reduces a
// contiguous pixel range in chunks of 128 pixels. A chunk's q and k head slices are read with
// 16-byte loads (8 channels of one pixel per lane, coalesced) one chunk AHEAD into registers,
// written transposed into LDS ([channel][pixel]), and each wave contracts its 32 pixels with
// MFMA:
//   cross blocks  Q^T K  (NB x NB blocks of 16 x 16)
//   diagonal blocks of Q^T Q and K^T K, whose diagonals are the squared norms.
// bf16 inputs use bf16 MFMA (products exact in fp32), fp32 inputs fp32 MFMA. The 4 waves'
// partials are summed in LDS (the transpose tile's memory, reused) in a fixed order and
// written to scratch as one record per split.
// Stage 2 (gram_reduce_kernel): RS slices of the splits summed per element, in split order.
// Stage 3 (gram_finish_kernel), one workgroup per (image, head): sums the RS slices in order,
// scales by rsqrt(max(|.|^2, 1e-24)) and the temperature, and applies a row softmax.
// The result is deterministic (fixed summation order for a given shape).
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

template <int NB, int DT>
__host__ __device__ constexpr int gram_lds_bytes() {
  // max(transpose tile, 4-wave reduction buffer)
  return (2 * NB * 16 * (GP_CHUNK + (DT == DT_BF16 ? 8 : 4)) * (DT == DT_BF16 ? 2 : 4)) >
                 (4 * (NB * 16 * NB * 16 + 2 * NB * 16) * 4)
             ? (2 * NB * 16 * (GP_CHUNK + (DT == DT_BF16 ? 8 : 4)) * (DT == DT_BF16 ? 2 : 4))
             : (4 * (NB * 16 * NB * 16 + 2 * NB * 16) * 4);
}

template <int NB, int DT>
__global__ void __launch_bounds__(256) gram_partial_kernel(const void* __restrict__ qkv, float* __restrict__ part,
                                                           int64_t hw, int c, int ch, int heads,
                                                           int64_t split_len, int nsplit) {
  constexpr int CP = NB * 16;                               // padded head channels
  constexpr int ES = (DT == DT_BF16) ? 2 : 4;
  constexpr int TROW = GP_CHUNK + (DT == DT_BF16 ? 8 : 4);  // LDS row (elements), +16 B
  constexpr int REC = CP * CP + 2 * CP;
  constexpr int UPT = (GP_CHUNK * 2 * 8 + 255) / 256;       // 16-byte units per thread (<= 8 groups)
  __shared__ __attribute__((aligned(16))) unsigned char smem[gram_lds_bytes<NB, DT>()];
  unsigned char* tl = smem;                                 // rows [0, CP) q, [CP, 2 CP) k
  float* red = reinterpret_cast<float*>(smem);              // reused after the pixel loop

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lc = lane & 15, lg = lane >> 4;
  const int nh = blockIdx.y;
  const int img = nh / heads, hd = nh - img * heads;
  const int64_t p_begin = (int64_t)blockIdx.x * split_len;
  int64_t p_end = p_begin + split_len;
  if (p_end > hw) p_end = hw;
  const int64_t row_stride = 3LL * c;  // elements per pixel
  const unsigned char* base = (const unsigned char*)qkv + (int64_t)img * hw * row_stride * ES;
  const int qoff = hd * ch, koff = c + hd * ch;
  const int groups = ch / 8;           // 8-channel groups per head slice
  const int units = GP_CHUNK * 2 * groups;

  // zero the padded channel rows once (they are never written by the loads)
  for (int u = tid; u < 2 * (CP - ch) * TROW; u += 256) {
    const int r = u / TROW, px = u - r * TROW;
    const int which = r / (CP - ch), rr = r - which * (CP - ch);
    const int row = which * CP + ch + rr;
    if constexpr (DT == DT_BF16) reinterpret_cast<unsigned short*>(tl)[row * TROW + px] = 0;
    else reinterpret_cast<float*>(tl)[row * TROW + px] = 0.f;
  }

  f32x4 cross[NB][NB], dq[NB], dk[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    dq[i] = dk[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NB; ++j) cross[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  u32x4 rq[UPT], rq2[DT == DT_F32 ? UPT : 1];
  auto fetch = [&](int64_t p0) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < UPT; ++j) {
      const int u = tid + j * 256;
      rq[j] = u32x4{0u, 0u, 0u, 0u};
      if constexpr (DT == DT_F32) rq2[j] = u32x4{0u, 0u, 0u, 0u};
      if (u < units) {
        const int px = u / (2 * groups);
        const int r = u - px * 2 * groups;
        const int which = r / groups;
        const int g = r - which * groups;
        const int64_t p = p0 + px;
        if (p < p_end) {
          const unsigned char* src = base + (p * row_stride + (which ? koff : qoff) + g * 8) * ES;
          rq[j] = *reinterpret_cast<const u32x4*>(src);
          if constexpr (DT == DT_F32) rq2[j] = *reinterpret_cast<const u32x4*>(src + 16);
        }
      }
    }
  };
  auto store_t = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < UPT; ++j) {
      const int u = tid + j * 256;
      if (u < units) {
        const int px = u / (2 * groups);
        const int r = u - px * 2 * groups;
        const int which = r / groups;
        const int g = r - which * groups;
        const int row0 = which * CP + g * 8;
        if constexpr (DT == DT_BF16) {
          unsigned short* t = reinterpret_cast<unsigned short*>(tl);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            t[(row0 + 2 * i) * TROW + px] = (unsigned short)(rq[j][i] & 0xffffu);
            t[(row0 + 2 * i + 1) * TROW + px] = (unsigned short)(rq[j][i] >> 16);
          }
        } else {
          float* t = reinterpret_cast<float*>(tl);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            t[(row0 + i) * TROW + px] = __uint_as_float(rq[j][i]);
            t[(row0 + 4 + i) * TROW + px] = __uint_as_float(rq2[j][i]);
          }
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
    // ---- this wave's 32 pixels: k = wave * 32 + 8 * lg + s
    const int kcol = wave * 32 + lg * 8;
    if constexpr (DT == DT_BF16) {
      bf16x8 qf[NB], kf[NB];
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        qf[i] = *reinterpret_cast<const bf16x8*>(tl + ((size_t)(i * 16 + lc) * TROW + kcol) * 2);
        kf[i] = *reinterpret_cast<const bf16x8*>(tl + ((size_t)(CP + i * 16 + lc) * TROW + kcol) * 2);
      }
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        dq[i] = mfma_bf16(qf[i], qf[i], dq[i]);
        dk[i] = mfma_bf16(kf[i], kf[i], dk[i]);
#pragma unroll
        for (int j = 0; j < NB; ++j) cross[i][j] = mfma_bf16(qf[i], kf[j], cross[i][j]);
      }
    } else {
      f32x8 qf[NB], kf[NB];
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const float* ra = reinterpret_cast<const float*>(tl) + (i * 16 + lc) * TROW + kcol;
        const float* rb = reinterpret_cast<const float*>(tl) + (CP + i * 16 + lc) * TROW + kcol;
        const f32x4 a0 = *reinterpret_cast<const f32x4*>(ra), a1 = *reinterpret_cast<const f32x4*>(ra + 4);
        const f32x4 b0 = *reinterpret_cast<const f32x4*>(rb), b1 = *reinterpret_cast<const f32x4*>(rb + 4);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          qf[i].v[s] = a0[s]; qf[i].v[4 + s] = a1[s];
          kf[i].v[s] = b0[s]; kf[i].v[4 + s] = b1[s];
        }
      }
#pragma unroll
      for (int i = 0; i < NB; ++i) {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          dq[i] = mfma_f32(qf[i].v[s], qf[i].v[s], dq[i]);
          dk[i] = mfma_f32(kf[i].v[s], kf[i].v[s], dk[i]);
#pragma unroll
          for (int j = 0; j < NB; ++j) cross[i][j] = mfma_f32(qf[i].v[s], kf[j].v[s], cross[i][j]);
        }
      }
    }
  }

  // ---- reduce the 4 waves (fixed order) and write this split's record
  // D layout: lane holds rows 4*lg + r (q channel within block i), column lc (k channel)
  __syncthreads();  // the transpose tile is free: reuse it as the reduction buffer
  float* my = red + wave * REC;
#pragma unroll
  for (int i = 0; i < NB; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int qi = i * 16 + lg * 4 + r;
#pragma unroll
      for (int j = 0; j < NB; ++j) my[qi * CP + j * 16 + lc] = cross[i][j][r];
      if (lg * 4 + r == lc) {  // diagonal element of the Q^T Q / K^T K block
        my[CP * CP + qi] = dq[i][r];
        my[CP * CP + CP + qi] = dk[i][r];
      }
    }
  }
  __syncthreads();
  float* out = part + ((int64_t)nh * nsplit + blockIdx.x) * REC;
  for (int e = tid; e < REC; e += 256)
    out[e] = ((red[e] + red[REC + e]) + red[2 * REC + e]) + red[3 * REC + e];
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
  for (int sp = s0; sp < s1; ++sp) s += src[(int64_t)sp * rec];
  part2[((int64_t)nh * GP_RS + sl) * rec + e] = s;
}

template <int NB>
__global__ void __launch_bounds__(256) gram_finish_kernel(const float* __restrict__ part2, const float* __restrict__ temp,
                                                          float* __restrict__ out, int ch, int heads) {
  constexpr int CP = NB * 16;
  constexpr int REC = CP * CP + 2 * CP;
  __shared__ float g[CP * CP];
  __shared__ float nq[CP], nk[CP];
  const int nh = blockIdx.x;
  const int hd = nh % heads;
  const float* src = part2 + (int64_t)nh * GP_RS * REC;
  for (int e = threadIdx.x; e < REC; e += 256) {
    float s = 0.f;
#pragma unroll
    for (int sl = 0; sl < GP_RS; ++sl) s += src[sl * REC + e];
    if (e < CP * CP) g[e] = s;
    else if (e < CP * CP + CP) nq[e - CP * CP] = rsqrtf(fmaxf(s, 1e-24f));
    else nk[e - CP * CP - CP] = rsqrtf(fmaxf(s, 1e-24f));
  }
  __syncthreads();
  const float t = temp[hd];
  // one wave per row: softmax over the ch columns
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int i = wave; i < ch; i += 4) {
    float v = -INFINITY;
    if (lane < ch) v = g[i * CP + lane] * nq[i] * nk[lane] * t;
    float mx = v;
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    const float e = (lane < ch) ? expf(v - mx) : 0.f;
    float s = e;
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if (lane < ch) out[((int64_t)nh * ch + i) * ch + lane] = e / s;
  }
}

static int pick_nb(int64_t ch) { return (int)((ch + 15) / 16); }

static int64_t split_len_for(int64_t batch, int64_t heads, int64_t hw) {
  // ~1024 workgroups in total, whole chunks per split
  int64_t want = (1024 + batch * heads - 1) / (batch * heads);
  if (want < 1) want = 1;
  int64_t len = (hw + want - 1) / want;
  len = (len + GP_CHUNK - 1) / GP_CHUNK * GP_CHUNK;
  return len < GP_CHUNK ? GP_CHUNK : len;
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
  CLARUS_REQUIRE(qkv && temperature && out && scratch, "channel_attention: null operand");
  CLARUS_REQUIRE(batch > 0 && hw > 0 && c > 0 && heads > 0 && c % heads == 0, "channel_attention: bad sizes");
  CLARUS_REQUIRE(qkv_dtype == DT_BF16 || qkv_dtype == DT_F32, "channel_attention: bad dtype");
  const int64_t ch = c / heads;
  CLARUS_REQUIRE(ch % 8 == 0 && ch <= 64, "channel_attention: head width %lld must be a multiple of 8, <= 64",
                 (long long)ch);
  CLARUS_REQUIRE(aligned(qkv, 16) && (c * (qkv_dtype == DT_BF16 ? 2 : 4)) % 16 == 0,
                 "channel_attention: qkv rows must be 16-byte aligned");
  const size_t need = clarus_hip_channel_attention_workspace(batch, hw, c, heads);
  CLARUS_REQUIRE(scratch_bytes >= need, "channel_attention: scratch %zu < %zu bytes", scratch_bytes, need);
  const int64_t len = split_len_for(batch, heads, hw);
  const int nsplit = (int)cdiv(hw, len);
  const int nb = pick_nb(ch);
  const int64_t rec = gram_rec_floats(nb);
  hipStream_t s = (hipStream_t)stream;
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
  switch (nb) {
    case 1: CLARUS_GRAM(1); break;
    case 2: CLARUS_GRAM(2); break;
    case 3: CLARUS_GRAM(3); break;
    default: CLARUS_GRAM(4); break;
  }
#undef CLARUS_GRAM
  return check_launch("channel_attention");
}
