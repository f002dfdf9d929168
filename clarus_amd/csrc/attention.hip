// Restormer MDTA attention map on gfx950:
//   A[n, hd] = softmax( (q / |q|) (k / |k|)^T * t[hd] ),  q, k: [HW, c_h] head slices of qkv.
//
// One launch, gram_kernel, one workgroup per (image, split, head), 256 threads.
// Pixel phase: each workgroup reduces a contiguous pixel range (a split) in chunks of 128
// pixels. A thread owns one unit of every chunk: 8 consecutive pixels x one 16-byte channel group
// of q or k (two units for fp32), loaded one chunk ahead through a buffer descriptor whose range
// ends at the split's end, so every load is issued and reads past the end return zero.
// A unit's squares feed the norms (fp32 VALU); the unit is transposed in registers and written
// as 8 rows of 16 bytes into the LDS tile [channel][pixel] (no bank conflicts). Each wave then
// contracts its 32 pixels with MFMA: the cross blocks Q^T K (NB x NB blocks of 16 x 16). bf16
// inputs use one bf16 MFMA per block (products exact in fp32); fp32 inputs are split into bf16
// hi + lo and use three (hi hi + hi lo + lo hi, error <= 2^-16 relative per product). The 4
// waves' partials are summed in LDS in a fixed order and written as the split's record.
// Reduction, in the same launch, up a tree of fan-in CA_FAN over the splits of an (image, head):
// after its record is stored (device-scope stores, complete before the arrival), a workgroup
// counts its arrival at its tree node; the last of the node's children to arrive sums their
// records in child order (every load issued before the first add) and carries the sum one
// level up. The last arrival at the root holds the sums: it scales by rsqrt(max(|.|^2, 1e-24))
// and the temperature and applies the row softmax. Nothing waits for another workgroup, and
// every sum has one order whoever performs it, so the result is deterministic. The arrival
// counters sit at the start of the scratch: zero when a call starts, reset to zero by the
// workgroups that saw them complete.
#include <mutex>

#include "capi.hpp"
#include "common.hpp"

namespace clarus {

constexpr int GP_CHUNK = 128;                                  // pixels per chunk (32 per wave)
constexpr int CA_FAN = 8;                                      // records summed per tree node
constexpr int CA_COUNTERS = 16384;                             // arrival counters per scratch
constexpr int CA_MAX_NH = 496;                                 // (image, head) pairs per launch, at most
constexpr int64_t CA_COUNTER_BYTES = (int64_t)CA_COUNTERS * 4;

// record per (image*head, split): [NB*16][NB*16] cross, [NB*16] |q|^2, [NB*16] |k|^2
__host__ __device__ inline int64_t gram_rec_floats(int nb) {
  const int cp = nb * 16;
  return (int64_t)cp * cp + 2 * cp;
}

// LDS: the transposed chunk [2 CP rows][GP_CHUNK pixels] (+16 B per row), reused after the
// pixel loop as the 4-wave reduction buffer and the running sums of the reduction
template <int NB, int DT>
__host__ __device__ constexpr int gram_lds_bytes() {
  return (2 * NB * 16 * (GP_CHUNK * (DT == DT_BF16 ? 2 : 4) + 16)) > (4 * (NB * 16 * NB * 16 + 2 * NB * 16) * 4)
             ? (2 * NB * 16 * (GP_CHUNK * (DT == DT_BF16 ? 2 : 4) + 16))
             : (4 * (NB * 16 * NB * 16 + 2 * NB * 16) * 4);
}

// The reduction tree of one (image, head): level 0 holds the nsplit split records, level l + 1
// one record per group of CA_FAN consecutive level-l records; the level with one node is the
// result. tree_nodes(n) = records of all levels, tree_counters(n) = nodes above level 0.
__host__ __device__ inline int tree_nodes(int n) {
  int t = n;
  while (n > 1) {
    n = (n + CA_FAN - 1) / CA_FAN;
    t += n;
  }
  return t;
}
__host__ __device__ inline int tree_counters(int n) { return n > 1 ? tree_nodes(n) - n : 1; }

struct GramP {
  const void* qkv;
  float* part;          // [nh][tree_nodes(nsplit)][rec]: level 0 (the splits), then each level up
  unsigned* cnt;        // [nh][tree_counters(nsplit)]: one arrival counter per node above level 0
  const float* temp;    // [heads]
  float* out;           // [nh][ch][ch]
  int64_t hw, split_len;
  int c, ch, heads, nsplit, nimg;
};

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

// Records are exchanged between workgroups through device-scope accesses: stores written
// through to the device's point of coherence and loads that miss the per-CU and per-XCD caches
// (cache policy SC1), so no cache-wide writeback or invalidate is needed between them.
constexpr int CA_SC1 = 1 << 4;  // cache-policy operand of the raw buffer loads / stores: SC1

// dst[e] (LDS, e < REC) = sum over records r = 0 .. count - 1 (count <= CA_FAN) of
// rec[r * REC + e] (records at record index r0 of rs, a descriptor whose range is exactly
// rs_bytes), in record order (the first record added to zero); every load issued before the
// first add. Lanes without a slot, and records past count, load at offset rs_bytes, past the
// range, and read zero.
template <int REC>
__device__ __forceinline__ void sum_records(__amdgpu_buffer_rsrc_t rs, uint32_t rs_bytes, int r0, int count,
                                            float* dst, int tid) {
  static_assert(REC % 4 == 0, "records of whole 16-byte groups");
  constexpr int SLOTS = REC / 4;
  constexpr int PER = (SLOTS + 255) / 256;
  f32x4 v[CA_FAN][PER];
#pragma unroll
  for (int j = 0; j < CA_FAN; ++j)
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e4 = tid + 256 * i;
      const uint32_t o = (e4 < SLOTS && j < count) ? (uint32_t)(((r0 + j) * REC + e4 * 4) * 4) : rs_bytes;
      v[j][i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)o, 0, CA_SC1));
    }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < CA_FAN; ++j)
      if (j < count) acc += v[j][i];
    const int e4 = tid + 256 * i;
    if (e4 < SLOTS) *reinterpret_cast<f32x4*>(dst + e4 * 4) = acc;
  }
}

// record index r of rs = src[0 .. REC) (LDS), device-scope stores
template <int REC>
__device__ __forceinline__ void store_record(__amdgpu_buffer_rsrc_t rs, int r, const float* src, int tid) {
  for (int e4 = tid; e4 < REC / 4; e4 += 256)
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, *reinterpret_cast<const f32x4*>(src + e4 * 4)),
                                           rs, (r * REC + e4 * 4) * 4, 0, CA_SC1);
}

// One arrival on *counter by this workgroup, after every wave's device-scope record stores have
// completed: true in every thread of the workgroup that arrived last of `members`, which also
// resets the counter for the next call
__device__ __forceinline__ bool arrive_last(unsigned* counter, unsigned members, int* flag, int tid) {
  wait_vmcnt<0>();  // this wave's record stores are complete (written through)
  __syncthreads();
  if (tid == 0) {
    const unsigned old = atomicAdd(counter, 1u);
    *flag = old == members - 1u;
    if (old == members - 1u) atomicExch(counter, 0u);  // every member has arrived: the next call starts at zero
  }
  __syncthreads();
  return *flag != 0;
}

template <int NB, int DT>
__global__ void __launch_bounds__(256) gram_kernel(GramP p) {
  constexpr int CP = NB * 16;                      // padded head channels
  constexpr int ES = (DT == DT_BF16) ? 2 : 4;
  constexpr int CG = (DT == DT_BF16) ? 8 : 4;      // channels per 16-byte load
  constexpr int TROWB = GP_CHUNK * ES + 16;        // LDS row bytes (+16 B pad)
  constexpr int REC = CP * CP + 2 * CP;
  constexpr int OCT = GP_CHUNK / 8;                // 8-pixel octets per chunk
  __shared__ __attribute__((aligned(16))) unsigned char smem[gram_lds_bytes<NB, DT>()];
  __shared__ int s_flag;
  unsigned char* tl = smem;                        // rows [0, CP) q, [CP, 2 CP) k
  float* red = reinterpret_cast<float*>(smem);     // reused after the pixel loop

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lc = lane & 15, lg = lane >> 4;
  // XCD-aware order: workgroup L runs on XCD L % 8; the heads of one (image, split) are workgroups
  // L, L + 8, L + 16, ... of one XCD, dispatched back to back, so the 128-byte lines that heads
  // share (a pixel row holds every head's q and k channels) come from HBM into one L2 once.
  // Workgroups past the last split of a row of 8 have nothing to do.
  const int L = blockIdx.x, xcd = L & 7, r8 = L >> 3;
  const int hd = r8 % p.heads, sblk = r8 / p.heads;
  const int is = sblk * 8 + xcd;            // (image, split) index
  const int img = is / p.nsplit, split = is - img * p.nsplit;
  if (img >= p.nimg) return;
  const int nh = img * p.heads + hd;
  const int ch = p.ch;
  const int64_t p_begin = (int64_t)split * p.split_len;
  const int64_t p_end = p_begin + p.split_len < p.hw ? p_begin + p.split_len : p.hw;
  const int64_t len = p_end - p_begin;
  const int64_t row_bytes = 3LL * p.c * ES;
  // the split's rows as a buffer range: loads at or past the split's end read zero
  const uint32_t nbytes = (uint32_t)(len * row_bytes);
  const __amdgpu_buffer_rsrc_t rs =
      buf_rsrc_n((const unsigned char*)p.qkv + ((int64_t)img * p.hw + p_begin) * row_bytes, nbytes);
  const int groups = ch / CG;          // load groups per head slice
  // units of a chunk: u = tid + 256 t = (which, group) * OCT + octet, octets in consecutive
  // lanes; 2 * groups * OCT <= 256 * UPT (head width <= 64)
  constexpr int UPT = (DT == DT_BF16) ? 1 : 2;
  int octet[UPT], row0[UPT];
  bool active[UPT];
  uint32_t uoff[UPT];  // byte offset of the unit's first pixel in chunk 0 (past the range: inactive)
#pragma unroll
  for (int t = 0; t < UPT; ++t) {
    const int u = tid + 256 * t;
    octet[t] = u % OCT;
    const int wg_ = u / OCT;
    active[t] = wg_ < 2 * groups;
    const int which = active[t] ? wg_ / groups : 0;
    const int grp = active[t] ? wg_ - which * groups : 0;
    const int64_t coff = (which ? p.c : 0) + hd * ch + grp * CG;  // channel offset of the unit
    row0[t] = which * CP + grp * CG;                             // its first LDS row
    uoff[t] = active[t] ? (uint32_t)(octet[t] * 8 * row_bytes + coff * ES) : 0x80000000u;
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

  // chunk starting at pixel r0 of the split into r (every load issued; inactive units and
  // pixels past the split read zero)
  auto fetch = [&](u32x4 (&r)[UPT][8], int64_t r0) __attribute__((always_inline)) {
    const uint32_t cb = (uint32_t)(r0 * row_bytes);
#pragma unroll
    for (int t = 0; t < UPT; ++t)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t o = uoff[t] + cb + (uint32_t)(i * row_bytes);
        r[t][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)o, 0, 0));
      }
  };
  auto store_t = [&](const u32x4 (&rq)[UPT][8]) __attribute__((always_inline)) {
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
  // this wave's 32 pixels of the tile: k = wave * 32 + 8 lg + s
  auto products = [&]() __attribute__((always_inline)) {
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
  };

  // pixel loop: the next chunk loads while this one is transposed and contracted (a chunk past
  // the split's end reads zero and adds nothing). Measured against two chunks in flight per
  // thread (a second register buffer, barriers that keep loads outstanding): equal or slower.
  u32x4 ra[UPT][8];
  fetch(ra, 0);
  for (int64_t r0 = 0; r0 < len; r0 += GP_CHUNK) {
    __syncthreads();  // the previous chunk's fragment reads are done
    store_t(ra);
    __syncthreads();
    fetch(ra, r0 + GP_CHUNK);
    products();
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
  const int nrec = tree_nodes(p.nsplit);
  const uint32_t recs_bytes = (uint32_t)(nrec * REC * 4);  // this (image, head)'s records
  const __amdgpu_buffer_rsrc_t recs = buf_rsrc_n(p.part + (int64_t)nh * nrec * REC, recs_bytes);
  {
    // the 4 waves' cross blocks summed in wave order into wave 0's slot (norms already there)
    for (int e = tid; e < CP * CP; e += 256) red[e] = ((red[e] + red[REC + e]) + red[2 * REC + e]) + red[3 * REC + e];
    __syncthreads();
    store_record<REC>(recs, split, red, tid);
  }

  // ---- the reduction over splits, up the tree: the last arrival at a node sums its (up to
  // CA_FAN) children in order and carries on one level up; the last at the root has the sums
  unsigned* cnt = p.cnt + (int64_t)nh * tree_counters(p.nsplit);
  int n = p.nsplit, base = 0, cbase = 0, r = split;
  for (;;) {
    const int g = r / CA_FAN, c0 = g * CA_FAN;
    const int members = n - c0 < CA_FAN ? n - c0 : CA_FAN;
    if (!arrive_last(cnt + cbase + g, (unsigned)members, &s_flag, tid)) return;
    sum_records<REC>(recs, recs_bytes, base + c0, members, red, tid);
    const int up = (n + CA_FAN - 1) / CA_FAN;
    if (up == 1) break;  // the root: red holds this (image, head)'s sums
    __syncthreads();
    store_record<REC>(recs, base + n + g, red, tid);
    base += n;
    cbase += up;
    n = up;
    r = g;
  }
  __syncthreads();

  // ---- norms, temperature and the row softmax of this (image, head)
  float* nq = red + REC;
  float* nk = nq + CP;
  for (int e = tid; e < 2 * CP; e += 256) {
    const float s2 = red[CP * CP + e];
    if (e < CP) nq[e] = rsqrtf(fmaxf(s2, 1e-24f));
    else nk[e - CP] = rsqrtf(fmaxf(s2, 1e-24f));
  }
  __syncthreads();
  const float tt = p.temp[hd];
  // four threads per row, CP / 4 columns each (interleaved: column 4 m + q of thread q); max
  // and sum over the four lanes with two butterfly steps
  constexpr int CPT = CP / 4;
  const int i = tid >> 2, q = tid & 3;
  if (i < CP) {
    float v[CPT];
    float mx = -INFINITY;
    const float si = nq[i] * tt;
#pragma unroll
    for (int m = 0; m < CPT; ++m) {
      const int j = 4 * m + q;
      v[m] = (i < ch && j < ch) ? red[i * CP + j] * si * nk[j] : -INFINITY;
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
      float* o = p.out + ((int64_t)nh * ch + i) * ch;
#pragma unroll
      for (int m = 0; m < CPT; ++m)
        if (4 * m + q < ch) o[4 * m + q] = v[m] * inv;
    }
  }
}

static int pick_nb(int64_t ch) { return (int)((ch + 15) / 16); }

struct GramPlan {
  int64_t nh;         // (image, head) pairs per launch
  int64_t split_len;  // pixels per split (whole chunks)
  int nsplit;
};

// Splits: about 2 workgroups per CU over the launch (measured at the config-4 levels against 3
// and 4: fewer records to sum, same pixel rate; whole chunks, not rounded to pairs: l0 fp32 96.5
// -> 92.9 us), a split's bytes (plus the chunk read past it) addressable with 32-bit offsets.
// The (image, head) pairs of a launch are bounded by the counters their trees need.
static GramPlan gram_plan(int64_t batch, int64_t heads, int64_t hw, int64_t c) {
  GramPlan g;
  int64_t imgs = batch < CA_MAX_NH / heads ? batch : CA_MAX_NH / heads;
  const int64_t chunks = cdiv(hw, GP_CHUNK);
  const int64_t row_bytes = 3 * c * 4;  // fp32 rows: the same plan (and workspace) for both dtypes
  const int64_t want = cdiv(2LL * device_cus(), imgs * heads);
  int64_t per = cdiv(chunks, want);
  const int64_t max_per = ((int64_t)1 << 30) / (GP_CHUNK * row_bytes);
  if (per > max_per) per = max_per;
  if (per < 1) per = 1;
  g.split_len = per * GP_CHUNK;
  g.nsplit = (int)cdiv(hw, g.split_len);
  const int64_t per_nh = tree_counters(g.nsplit);
  if (imgs * heads * per_nh > CA_COUNTERS) imgs = CA_COUNTERS / (per_nh * heads);
  g.nh = (imgs < 1 ? 1 : imgs) * heads;
  return g;
}

static int64_t gram_workspace_bytes(const GramPlan& g, int64_t ch) {
  return CA_COUNTER_BYTES + g.nh * (int64_t)tree_nodes(g.nsplit) * gram_rec_floats(pick_nb(ch)) * 4;
}

// Launches gram_kernel per batch slice of at most CA_MAX_NH (image, head) pairs, with `scratch`
// as counters (zero on entry) + partials (already checked to be large enough).
static int launch_channel_attention(const void* qkv, int32_t qkv_dtype, const float* temperature, float* out,
                                    int64_t batch, int64_t hw, int64_t c, int64_t heads, void* scratch,
                                    hipStream_t s) {
  const int64_t ch = c / heads;
  const GramPlan g = gram_plan(batch, heads, hw, c);
  const int nb = pick_nb(ch);
  const int64_t imgs = g.nh / heads;
  const int64_t img_bytes = hw * 3 * c * (qkv_dtype == DT_BF16 ? 2 : 4);
  note_kernel("gram_kernel nb=%d nsplit=%d", nb, g.nsplit);
  for (int64_t i0 = 0; i0 < batch; i0 += imgs) {
    const int64_t ni = batch - i0 < imgs ? batch - i0 : imgs;
    GramP p;
    p.qkv = (const unsigned char*)qkv + i0 * img_bytes;
    p.cnt = (unsigned*)scratch;
    p.part = (float*)((unsigned char*)scratch + CA_COUNTER_BYTES);
    p.temp = temperature;
    p.out = out + i0 * heads * ch * ch;
    p.hw = hw;
    p.split_len = g.split_len;
    p.c = (int)c;
    p.ch = (int)ch;
    p.heads = (int)heads;
    p.nsplit = g.nsplit;
    p.nimg = (int)ni;
    dim3 grid((unsigned)(cdiv(ni * g.nsplit, 8) * 8 * heads));
#define CLARUS_GRAM(NB)                                                                                   \
  do {                                                                                                    \
    if (qkv_dtype == DT_BF16) hipLaunchKernelGGL((gram_kernel<NB, DT_BF16>), grid, dim3(256), 0, s, p);  \
    else hipLaunchKernelGGL((gram_kernel<NB, DT_F32>), grid, dim3(256), 0, s, p);                        \
  } while (0)
    switch (nb) {
      case 1: CLARUS_GRAM(1); break;
      case 2: CLARUS_GRAM(2); break;
      case 3: CLARUS_GRAM(3); break;
      default: CLARUS_GRAM(4); break;
    }
#undef CLARUS_GRAM
  }
  return check_launch("channel_attention");
}

static int check_channel_attention(const void* qkv, int32_t qkv_dtype, const float* temperature, const float* out,
                                   int64_t batch, int64_t hw, int64_t c, int64_t heads) {
  CLARUS_REQUIRE(qkv && temperature && out, "channel_attention: null operand");
  CLARUS_REQUIRE(batch > 0 && hw > 0 && c > 0 && heads > 0 && c % heads == 0, "channel_attention: bad sizes");
  CLARUS_REQUIRE(heads <= CA_MAX_NH, "channel_attention: at most %d heads", CA_MAX_NH);
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
  if (batch <= 0 || hw <= 0 || c <= 0 || heads <= 0 || c % heads || heads > CA_MAX_NH) return 0;
  return (size_t)gram_workspace_bytes(gram_plan(batch, heads, hw, c), c / heads);
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
