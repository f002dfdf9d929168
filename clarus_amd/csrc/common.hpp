// Device helpers shared by the gfx950 kernels of libclarus_hip.so.
//
// MFMA conventions used throughout (CDNA3/CDNA4 16x16 family, wave64, lane l):
//   D = A . B with A [16 x K], B [K x 16], D [16 x 16] fp32.
//   D:  lane l holds D[4 * (l / 16) + j][l % 16], j = 0..3.
//   A / B: lane l supplies row (A) / column (B) l % 16; the K values a lane supplies are
//   selected by l / 16. Both operands use the same K selection, so which physical k each
//   (lane, slot) pair stands for is free as long as A and B agree; the kernels load 8
//   consecutive k per lane (k = 8 * (l / 16) + i) for every instruction flavour:
//     bf16 16x16x32: slot i of the 8-vector is k = 8 * (l / 16) + i
//     fp32 16x16x4 : instruction i (of 8) uses slot i, covering k = 8 * (l / 16) + i
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace clarus {

typedef __bf16 bf16_t;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;
typedef __attribute__((ext_vector_type(2))) float f32x2;

enum : int { DT_F32 = 0, DT_BF16 = 1 };
enum : int { ACT_NONE = 0, ACT_GELU = 1, ACT_LRELU = 2 };

struct f32x8 {
  float v[8];
};

__device__ __forceinline__ float bf16_to_f32(unsigned short h) {
  return __uint_as_float(((unsigned int)h) << 16);
}

// round-to-nearest-even fp32 -> bf16 bits (torch's Tensor.to(bfloat16) rounding); NaN stays NaN
__device__ __forceinline__ unsigned short f32_to_bf16_bits(float f) {
  bf16_t b = (bf16_t)f;
  return __builtin_bit_cast(unsigned short, b);
}

// 8 consecutive elements at p (16-byte aligned for bf16, 32-byte for fp32) as fp32
template <int DT>
__device__ __forceinline__ f32x8 load8(const void* p) {
  f32x8 r;
  if constexpr (DT == DT_BF16) {
    u32x4 q = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r.v[2 * i] = __uint_as_float(q[i] << 16);
      r.v[2 * i + 1] = __uint_as_float(q[i] & 0xffff0000u);
    }
  } else {
    f32x4 a = reinterpret_cast<const f32x4*>(p)[0];
    f32x4 b = reinterpret_cast<const f32x4*>(p)[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r.v[i] = a[i];
      r.v[4 + i] = b[i];
    }
  }
  return r;
}

__device__ __forceinline__ f32x8 zero8() {
  f32x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r.v[i] = 0.f;
  return r;
}

__device__ __forceinline__ float load1(const void* p, int dt, int64_t i) {
  if (dt == DT_BF16) return bf16_to_f32(reinterpret_cast<const unsigned short*>(p)[i]);
  return reinterpret_cast<const float*>(p)[i];
}

__device__ __forceinline__ void store1(void* p, int dt, int64_t i, float v) {
  if (dt == DT_BF16)
    reinterpret_cast<unsigned short*>(p)[i] = f32_to_bf16_bits(v);
  else
    reinterpret_cast<float*>(p)[i] = v;
}

// sum over the G consecutive lanes of a group (G a power of two <= 64), xor butterfly 1 .. G / 2:
// the reduction order of the row prologues (clarus_hip_rows_prologue and the GEMMs that apply it
// to whole rows in LDS or registers), so their statistics agree bit for bit
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = 1; o < G; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// pack 8 fp32 into 8 bf16 (RNE)
__device__ __forceinline__ bf16x8 pack_bf16(const f32x8& a) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (bf16_t)a.v[i];
  return r;
}

// a = hi + lo with hi, lo bf16: |a - hi - lo| <= 2^-16 |a| (both roundings RNE)
__device__ __forceinline__ void split_bf16(const f32x8& a, bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    bf16_t h = (bf16_t)a.v[i];
    hi[i] = h;
    lo[i] = (bf16_t)(a.v[i] - (float)h);
  }
}

__device__ __forceinline__ f32x4 mfma_bf16(const bf16x8& a, const bf16x8& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Workgroup barrier that leaves outstanding global loads in flight. __syncthreads() is a
// workgroup fence plus s_barrier, and the fence makes every wave wait for all of its vector
// memory operations first (vmcnt(0)): that drains a prefetch or LDS-copy ring at each barrier.
// Callers of this barrier order their global -> LDS copies with explicit vmcnt waits; the
// wave's own LDS reads and writes are complete before it arrives (lgkmcnt(0)). The asm is also
// a compiler barrier for memory operations.
__device__ __forceinline__ void barrier_keep_vm() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// vmcnt(N) (expcnt / lgkmcnt untouched): the count's low 4 bits in [3:0], high 2 bits in [15:14]
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// A raw buffer descriptor for base address p (wave-uniform): 32-bit byte offsets from p, a
// range of 2^31 - 1 bytes, word 3 = 0x00020000 (32-bit data format, as CDNA's untyped buffer
// instructions need). Loads and stores through it take a scalar base and a VGPR offset.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, 0x7fffffff, 0x00020000);
}

// The same with a range of nbytes: loads at or past it read 0 and stores there are dropped, while
// every lane still issues the instruction (so vmcnt counts it whatever the row)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc_n(const void* p, uint32_t nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)nbytes, 0x00020000);
}

// exact-erf GELU (torch.nn.functional.gelu default)
__device__ __forceinline__ float gelu_erf(float x) {
  return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
}

// sum over the 4 lanes {l, l^16, l^32, l^48} (the lanes that share an MFMA column)
__device__ __forceinline__ float sum_col4(float v) {
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

__host__ __device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace clarus
