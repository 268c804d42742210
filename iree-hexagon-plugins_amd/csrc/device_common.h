// Device-side helpers shared by the gfx950 kernels: vector types, MFMA
// wrappers, direct global->LDS loads, wait counters and the XCD-aware
// workgroup order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ihp {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

#define IHP_LDS __attribute__((address_space(3)))

// One 32x32 MFMA over a 32-byte K slab per lane pair (16 bytes per lane):
//   f16: v_mfma_f32_32x32x16_f16  (K = 16 halves)
//   i8 : v_mfma_i32_32x32x32_i8   (K = 32 bytes)
// Operand lane layout: lane l supplies row (l % 32) and the 16-byte K chunk
// (l / 32) of the slab. The product pairs A and B elements at the same
// (lane group, element) position, so any K assignment used identically for
// A and B gives the same sum. Output: lane l holds column (l % 32); register r
// holds row 8*(r/4) + 4*(l/32) + (r%4).
template <typename T>
struct Mfma32;

template <>
struct Mfma32<f16> {
  typedef f32x16 Acc;
  typedef float AccScalar;
  static __device__ __forceinline__ Acc mma(i32x4 a, i32x4 b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(
        __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
        0);
  }
};

template <>
struct Mfma32<int8_t> {
  typedef i32x16 Acc;
  typedef int AccScalar;
  static __device__ __forceinline__ Acc mma(i32x4 a, i32x4 b, Acc c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
};

// 16x16 MFMA over a 64-byte K slab (16 bytes per lane, 4 lane groups):
//   f16: v_mfma_f32_16x16x32_f16, i8: v_mfma_i32_16x16x64_i8.
// Lane l supplies row (l % 16) and K chunk (l / 16). Output: lane l holds
// column (l % 16); register r holds row 4*(l/16) + r.
template <typename T>
struct Mfma16;

template <>
struct Mfma16<f16> {
  typedef f32x4 Acc;
  typedef float AccScalar;
  static __device__ __forceinline__ Acc mma(i32x4 a, i32x4 b, Acc c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(
        __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
        0);
  }
};

template <>
struct Mfma16<int8_t> {
  typedef i32x4 Acc;
  typedef int AccScalar;
  static __device__ __forceinline__ Acc mma(i32x4 a, i32x4 b, Acc c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
  }
};

// 16-byte direct global->LDS copy (global_load_lds_dwordx4). Lane i of the
// wave writes lds_wave_base + 16*i; lds_wave_base must be wave-uniform.
__device__ __forceinline__ void global_to_lds_16(const void *gptr,
                                                 IHP_LDS void *lds_wave_base) {
  __builtin_amdgcn_global_load_lds(gptr, lds_wave_base, 16, 0, 0);
}

// The same copy from a wave-uniform 64-bit base (SGPRs) plus a 32-bit
// per-lane offset, with the LDS address in M0 set from an SGPR: the
// global_load_lds saddr form. The address then costs no vector instruction;
// the builtin above makes the compiler build a 64-bit per-lane address and
// move the LDS address out of a VGPR (v_readfirstlane) for every copy.
// Issued as asm, so it is not counted by the compiler's own waits: callers
// wait with wait_vmcnt<N>().
__device__ __forceinline__ void global_to_lds_16s(const char *sbase,
                                                  uint32_t voff,
                                                  IHP_LDS void *lds_wave_base) {
  const uint32_t m0 = (uint32_t)(uintptr_t)lds_wave_base;
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(voff), "s"(sbase), "s"(m0)
      : "memory", "m0");
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt[3:0] | vmcnt[5:4] << 14, other
// counters left at their maximum so they are not waited on).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) |
                             (0xF << 8));
}

// Workgroup barrier without the memory fence __syncthreads() adds: the fence
// makes the compiler emit s_waitcnt vmcnt(0) first, which would drain every
// in-flight global->LDS prefetch. Callers wait on exactly the counters they
// need (wait_vmcnt / wait_lgkmcnt0) before it; the "memory" clobber keeps the
// compiler from moving memory accesses across it.
__device__ __forceinline__ void block_barrier() {
  asm volatile("s_barrier" ::: "memory");
}

__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4) | (0x0 << 8));
}

__device__ __forceinline__ i32x4 lds_read_16(const IHP_LDS char *p) {
  return *(const IHP_LDS i32x4 *)p;
}

// ds_read_b128 issued as inline asm: the compiler inserts no wait for it, so
// the caller must wait with lgkm_wait<N>() and tie the result registers with
// lgkm_tie() before using them. LDS reads return in issue order, so after
// issuing R more reads, lgkmcnt(R) guarantees this one has landed.
template <int OFF>
__device__ __forceinline__ i32x4 lds_read_16_async(const IHP_LDS char *p) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset range");
  i32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2"
               : "=v"(v)
               : "v"((unsigned)(uintptr_t)p), "i"(OFF));
  return v;
}

template <int N>
__device__ __forceinline__ void lgkm_wait() {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N));
}

// Orders every later use of `v` after the preceding lgkm_wait (both are
// volatile asm, which keep their order).
__device__ __forceinline__ void lgkm_tie(i32x4 &v) {
  asm volatile("" : "+v"(v));
}

// 16 bytes written through. The compiler's hazard pass does not see inline
// asm as a store, and on gfx950 a VALU write to the data registers of a
// store wider than 8 bytes needs two wait states after it: without the
// s_nop the compiler may reuse those registers at once and the store then
// writes the new values (seen as wrong, run-to-run varying C2 outputs in an
// experimental build; the shipped schedule had the slots by chance).
__device__ __forceinline__ void store_through16(void *p, i32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" ::"v"(p),
               "v"(v)
               : "memory");
}

// Device-scope (sc1) 32-bit store / load for data one workgroup publishes and
// another, possibly on another XCD, reads within the same kernel: the store
// is written through past this XCD's L2 and the load bypasses it. They are
// the instructions the compiler emits for agent-scope relaxed atomics, issued
// as asm so they are not each followed by a wait: callers drain stores with
// wait_vmcnt<0>() and collect loads with partial_sum().
__device__ __forceinline__ void store_device(float *p, float v) {
  asm volatile("global_store_dword %0, %1, off sc1" ::"v"(p), "v"(v)
               : "memory");
}
__device__ __forceinline__ void store_device(int *p, int v) {
  asm volatile("global_store_dword %0, %1, off sc1" ::"v"(p), "v"(v)
               : "memory");
}
template <typename P>
__device__ __forceinline__ P load_device(const P *p) {
  static_assert(sizeof(P) == 4, "32-bit");
  P v;
  asm volatile("global_load_dword %0, %1, off sc1" : "=v"(v) : "v"(p)
               : "memory");
  return v;
}
template <typename P>
__device__ __forceinline__ void vm_tie(P &v) {
  asm volatile("" : "+v"(v));
}

// sum_{s < splits} base[s * stride], added in s order, with up to B loads in
// flight per wait (a short last batch adds exact zeros, which leave the sum
// unchanged).
template <typename P, int B = 8>
__device__ __forceinline__ P partial_sum(const P *base, int64_t stride,
                                         int splits) {
  P sum = 0;
  for (int s = 0; s < splits; s += B) {
    P v[B];
#pragma unroll
    for (int u = 0; u < B; ++u)
      v[u] = s + u < splits ? load_device(base + (int64_t)(s + u) * stride)
                            : (P)0;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int u = 0; u < B; ++u) {
      vm_tie(v[u]);
      sum += v[u];
    }
  }
  return sum;
}

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own
// L2). Renumber them so that consecutive logical tile ids share an XCD, then
// walk tiles in GROUP_M-row bands so an XCD's tiles reuse the same A row
// panels and B column panels from its L2.
__device__ __forceinline__ void xcd_tile_order(int wg, int num_wg,
                                               int tiles_m, int tiles_n,
                                               int group_m, int *tm, int *tn) {
  constexpr int kXcds = 8;
  int logical = wg;
  if (num_wg % kXcds == 0)
    logical = (wg % kXcds) * (num_wg / kXcds) + wg / kXcds;
  int per_group = group_m * tiles_n;
  int group = logical / per_group;
  int first_m = group * group_m;
  int rows = tiles_m - first_m < group_m ? tiles_m - first_m : group_m;
  int in_group = logical - group * per_group;
  *tm = first_m + in_group % rows;
  *tn = in_group / rows;
}

// 8 int8 weights (two dwords) -> 8 f16, exact: each byte b becomes the f16
// with exponent 2^10 and mantissa (b ^ 0x80), i.e. 1024 + (b + 128), and
// subtracting 1152 leaves b. Two v_perm_b32 and one packed f16 subtract per
// four weights.
__device__ __forceinline__ i32x4 i8x8_to_f16x8(i32x2 q) {
  i32x4 out;
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const unsigned y = (unsigned)q[d] ^ 0x80808080u;
    const unsigned lo = __builtin_amdgcn_perm(0x64646464u, y, 0x05010400u);
    const unsigned hi = __builtin_amdgcn_perm(0x64646464u, y, 0x07030602u);
    const f16x2 bias = {(f16)1152.0f, (f16)1152.0f};
    out[2 * d] = __builtin_bit_cast(int, __builtin_bit_cast(f16x2, lo) - bias);
    out[2 * d + 1] =
        __builtin_bit_cast(int, __builtin_bit_cast(f16x2, hi) - bias);
  }
  return out;
}

}  // namespace ihp
