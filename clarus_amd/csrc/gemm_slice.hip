// W-slice GEMM (gfx950): clarus_hip_gemm's kernel for small plain bf16 problems with a long K,
//
//   out[m][n] = (A[m][:] . W[:][n] + bias[n]) * scale[n] * out_scale      (bf16 A and W)
//
// the NAFNet SCA GEMM on the TLC map among them (level 3 at 720p: M = 4859, K = N = 512). Such a
// problem has too few 128 x 128 output tiles to fill 256 CUs, and every K = 512 tile spends
// most of its time filling and draining a copy pipeline that never reaches a steady state.
//
// Here a workgroup (8 waves, one per CU) holds one slice of 64 output channels of W^T in LDS
// (64 rows x K bf16, 64 KiB at K = 512) and each wave computes whole 32-pixel units against it.
// A unit's A rows reach the wave's LDS slot in pieces of up to 128 k (8 KiB) by direct
// global -> LDS copies of whole row segments, the wave reads its fragments of a piece into
// registers and refills the slot with the next piece at once, so one piece is in flight while
// one is computed. The W rows are copied the same way, row by row. (Loading the fragments
// straight from global memory, 32 rows x 32 bytes per instruction, measured slower than the
// tiled kernels: 18.4 against 14-16 us at the SCA shape.) Both LDS arrays keep the 16-byte
// units of a row XOR-swizzled with the row index, so that the 32 rows a fragment read touches
// fall on distinct banks. Products on 32x32x16 MFMAs:
// Workgroup order is XCD-aware: workgroups are dealt to the 8 XCDs in turn, and the workgroups
// an XCD receives cover all slices of the same unit groups, so each A row is fetched into one
// L2 only.
// Replaces the same fused_gemm call as the other clarus_hip_gemm kernels
// (kernels/gemm.py:353-400; the SCA GEMM: models/nafnet/__init__.py:157).
#include "capi.hpp"
#include "gemm_lds_dispatch.hpp"
#include "gemm_mfma32.hpp"

namespace clarus {

namespace {

constexpr int GS_P = 32;  // pixels per unit
constexpr int GS_N = 64;  // output channels per workgroup
constexpr int GS_W = 8;   // waves per workgroup (two per SIMD)

// k per A piece, pieces per unit, bytes per piece, LDS bytes (W slice | tables | 4 slots)
__host__ __device__ constexpr int gs_pk(int ks) { return ks * 16 < 128 ? ks * 16 : 128; }
__host__ __device__ constexpr int gs_piece_bytes(int ks) { return GS_P * gs_pk(ks) * 2; }
__host__ __device__ constexpr int gs_lds_bytes(int ks) {
  return GS_N * ks * 16 * 2 + 2 * GS_N * 4 + GS_W * gs_piece_bytes(ks);
}

__device__ __forceinline__ int gs_row(int T, int r) {
  return 32 * T + 16 * (r >> 4) + 8 * ((r >> 2) & 1) + 4 * ((r >> 3) & 1) + (r & 3);
}

template <int KS, int CDT>
__global__ void __launch_bounds__(64 * GS_W, 1) gemm_slice_kernel(const GemmP p, int slices, int rounds) {
  constexpr int K = KS * 16;
  constexpr int UW = K / 8;                  // 16-byte units per W^T / A row
  constexpr int WM = (UW < 32 ? UW : 32) - 1;  // W row swizzle mask
  constexpr int PK = gs_pk(KS), PU = PK / 8, PS = PK / 16, NP = K / PK;
  constexpr int PB = gs_piece_bytes(KS);
  constexpr int CPA = PB / 1024;             // copy instructions per piece
  constexpr int WB = GS_N * K * 2;
  constexpr int EC = CDT == DT_BF16 ? 2 : 4;
  constexpr int NS = CDT == DT_BF16 ? 4 : 8;  // 16-byte stores per lane per unit
  static_assert(NS < 16 && PB % 1024 == 0 && (PU & (PU - 1)) == 0, "layout");
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  float* tab = reinterpret_cast<float*>(lds + WB);  // bias [64] | scale * out_scale [64]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int px = lane & 31, hf = lane >> 5;
  unsigned char* slot = lds + WB + 2 * GS_N * 4 + wave * PB;
  // workgroup L runs on XCD L % 8; its index i = L / 8 there picks the slice (i % slices) and
  // the unit group (i / slices) * 8 + L % 8, then every 8 * rounds-th group after it; wave w
  // takes unit w of each group
  const int L = (int)blockIdx.x, i = L >> 3;
  const int slice = i % slices;
  const int g0 = (i / slices) * 8 + (L & 7);
  const int gstep = 8 * rounds;
  const int nunits = (int)cdiv(p.m, GS_P);
  const int ngroups = (nunits + GS_W - 1) / GS_W;
  if (g0 >= ngroups) return;  // uniform over the workgroup
  const int first = g0 * GS_W + wave;
  const int nmine = first < nunits ? (nunits - 1 - first) / (gstep * GS_W) + 1 : 0;
  const int64_t n0 = (int64_t)slice * GS_N;

  // ---- W^T rows n0 .. n0 + 63 -> LDS, whole rows per copy; position (row, v) holds unit v ^ (row & WM)
  const unsigned char* Wt = (const unsigned char*)p.wt + n0 * K * 2;
  for (int c = wave; c < UW; c += GS_W) {
    const int pos = c * 64 + lane, row = pos / UW, v = pos - row * UW;
    const unsigned char* src = Wt + (row * K + (v ^ (row & WM)) * 8) * 2;
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)(lds + c * 1024), 16, 0, 0);
  }
  if (tid < GS_N) {
    tab[tid] = p.bias ? p.bias[n0 + tid] : 0.f;
    tab[GS_N + tid] = (p.scale ? p.scale[n0 + tid] : 1.f) * p.out_scale;
  }

  const unsigned char* A = (const unsigned char*)p.a;
  unsigned char* C = (unsigned char*)p.c;
  const int64_t rb = p.lda * 2, cb = p.ldc * EC;
  // piece t of the wave (unit t / NP, k from (t % NP) PK) -> the slot, through a buffer bounded
  // to the unit's valid rows (rows past M read as zeros); position (row, v) holds unit v ^ row
  auto issue = [&](int t) __attribute__((always_inline)) {
    const int64_t q0 = (int64_t)(first + (t / NP) * gstep * GS_W) * GS_P;
    const int rows = p.m - q0 < GS_P ? (int)(p.m - q0) : GS_P;
    const __amdgpu_buffer_rsrc_t r = buf_rsrc_n(A + q0 * rb, (uint32_t)(rows * rb));
    const int kb = (t % NP) * PK * 2;
#pragma unroll
    for (int c = 0; c < CPA; ++c) {
      const int pos = c * 64 + lane, row = pos / PU, v = pos - row * PU;
      const uint32_t off = row * (uint32_t)rb + kb + (v ^ (row & (PU - 1))) * 16;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(slot + c * 1024), 16,
                                               off, 0, 0, 0);
    }
  };
  if (nmine > 0) issue(0);
  __syncthreads();  // W, the tables and each wave's first piece are in LDS
  if (nmine == 0) return;

  f32x16 acc[2];
  const int total = nmine * NP;
  for (int t = 0; t < total; ++t) {
    const int h = t % NP;
    // piece t was issued one iteration ago; after it only the last unit's NS stores (h == 0)
    if (t > 0) {
      if (h == 0) wait_vmcnt<NS>();
      else wait_vmem_all();
    }
    asm volatile("" ::: "memory");  // slot reads follow the wait
    u32x4 xr[PS];
#pragma unroll
    for (int s = 0; s < PS; ++s)
      xr[s] = *reinterpret_cast<const u32x4*>(slot + (px * PU + ((2 * s + hf) ^ (px & (PU - 1)))) * 16);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slot is free
    if (t + 1 < total) issue(t + 1);
    if (h == 0) {
#pragma unroll
      for (int T = 0; T < 2; ++T)
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const f32x4 b0 = *reinterpret_cast<const f32x4*>(tab + 32 * T + 16 * r + 8 * hf);
          const f32x4 b1 = *reinterpret_cast<const f32x4*>(tab + 32 * T + 16 * r + 8 * hf + 4);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            acc[T][8 * r + j] = b0[j];
            acc[T][8 * r + 4 + j] = b1[j];
          }
        }
    }
#pragma unroll
    for (int s = 0; s < PS; ++s) {
      const int u = 2 * (h * PS + s) + hf;  // this lane's 16-byte unit of the W row
#pragma unroll
      for (int T = 0; T < 2; ++T) {
        const int row = gs_row(T, px);
        const bf16x8 w = *reinterpret_cast<const bf16x8*>(lds + (row * UW + (u ^ (row & WM))) * 16);
        acc[T] = mfma32_bf16(w, __builtin_bit_cast(bf16x8, xr[s]), acc[T]);
      }
      // keep the scheduler from hoisting every W fragment of the piece at once
      if ((s & 3) == 3) __builtin_amdgcn_sched_barrier(0);
    }
    if (h == NP - 1) {
      const int64_t q0 = (int64_t)(first + (t / NP) * gstep * GS_W) * GS_P;
      const int rows = p.m - q0 < GS_P ? (int)(p.m - q0) : GS_P;
      const __amdgpu_buffer_rsrc_t orr = buf_rsrc_n(C + q0 * cb, (uint32_t)(rows * cb));
#pragma unroll
      for (int T = 0; T < 2; ++T)
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int ch = 32 * T + 16 * r + 8 * hf;
          const f32x4 s0 = *reinterpret_cast<const f32x4*>(tab + GS_N + ch);
          const f32x4 s1 = *reinterpret_cast<const f32x4*>(tab + GS_N + ch + 4);
          float v[8];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            v[j] = acc[T][8 * r + j] * s0[j];
            v[4 + j] = acc[T][8 * r + 4 + j] * s1[j];
          }
          const int off = px * (int)cb + (int)(n0 + ch) * EC;
          if constexpr (CDT == DT_BF16) {
            u32x4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j)
              o[j] = (unsigned)f32_to_bf16_bits(v[2 * j]) | ((unsigned)f32_to_bf16_bits(v[2 * j + 1]) << 16);
            __builtin_amdgcn_raw_buffer_store_b128(o, orr, off, 0, 0);
          } else {
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, f32x4{v[0], v[1], v[2], v[3]}), orr,
                                                   off, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, f32x4{v[4], v[5], v[6], v[7]}), orr,
                                                   off + 16, 0, 0);
          }
        }
    }
  }
  wait_vmem_all();
}

template <int KS, int CDT>
void launch_slice(const GemmP& p, int slices, int rounds, int64_t grid, hipStream_t s) {
  const int lds = gs_lds_bytes(KS);
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_slice_kernel<KS, CDT>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    attr = true;
  }
  hipLaunchKernelGGL((gemm_slice_kernel<KS, CDT>), dim3((unsigned)grid), dim3(64 * GS_W), lds, s, p, slices,
                     rounds);
}

}  // namespace

bool gemm_slice_fits(const GemmP& p) {
  return (p.k == 128 || p.k == 256 || p.k == 512) && p.n % GS_N == 0 && p.n / GS_N < (1 << 20) &&
         (p.c_dt == DT_BF16 || p.c_dt == DT_F32) && p.vec_out == 2 && p.lda * 2 * GS_P < ((int64_t)1 << 31) &&
         p.ldc * 4 * GS_P < ((int64_t)1 << 31) && cdiv(p.m, GS_P) < ((int64_t)1 << 30);
}

bool launch_gemm_slice(const GemmP& p, hipStream_t s) {
  if (!gemm_slice_fits(p)) return false;
  const int slices = (int)(p.n / GS_N);
  const int64_t ngroups = cdiv(cdiv(p.m, GS_P), GS_W);
  const int ks = (int)(p.k / 16);
  // one unit group per workgroup while the resident workgroups hold them all, else each
  // workgroup takes every (8 * rounds)-th group
  const int64_t per_cu = std::max(1, (160 * 1024) / gs_lds_bytes(ks));
  const int64_t rounds =
      std::max<int64_t>(1, std::min<int64_t>(cdiv(ngroups, 8), (per_cu * device_cus()) / (8LL * slices)));
  const int64_t grid = 8LL * slices * rounds;
  if (grid >= ((int64_t)1 << 31)) return false;
  if (p.c_dt == DT_BF16) {
    if (ks == 8) launch_slice<8, DT_BF16>(p, slices, (int)rounds, grid, s);
    else if (ks == 16) launch_slice<16, DT_BF16>(p, slices, (int)rounds, grid, s);
    else launch_slice<32, DT_BF16>(p, slices, (int)rounds, grid, s);
  } else {
    if (ks == 8) launch_slice<8, DT_F32>(p, slices, (int)rounds, grid, s);
    else if (ks == 16) launch_slice<16, DT_F32>(p, slices, (int)rounds, grid, s);
    else launch_slice<32, DT_F32>(p, slices, (int)rounds, grid, s);
  }
  return true;
}

}  // namespace clarus
