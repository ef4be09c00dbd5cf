// Wave-level helpers shared by the gfx950 kernels: wait counters, barriers,
// lane ids, DPP scans, transposing LDS reads and cross-lane reductions.
#pragma once

#include <utility>

#include "fa_common.h"

namespace fa {

// Load through the scalar unit (constant address space): for wave-uniform
// metadata, so the value arrives via lgkmcnt and never forces a vmcnt wait on
// the tile copies in flight.
template <typename T>
__device__ inline T sload(const T* p) {
  return *(const __attribute__((address_space(4))) T*)(p);
}

__device__ inline void wait_lds() { __builtin_amdgcn_s_waitcnt(0xC07F); }  // lgkmcnt(0)
// s_waitcnt lgkmcnt(N): all but the last N LDS operations done (LDS operations
// complete in order; only valid while no scalar load is outstanding)
template <int N>
__device__ inline void wait_lds_upto() {
  static_assert(N >= 0 && N <= 15, "lgkmcnt is four bits");
  __builtin_amdgcn_s_waitcnt(0xC07F | (N << 8));
}
// Work-group barrier that also fences the instruction scheduler: the phases
// between barriers are laid out by hand, so nothing may move across.
__device__ inline void barrier() {
  __builtin_amdgcn_sched_barrier(0);
  wait_lds();
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}
// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt low bits [3:0], high bits [15:14]).
template <int N>
__device__ inline void wait_vmem() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// Inclusive prefix sum over the 64 lanes of a wave by DPP (no LDS round trips):
// row shifts by 1, 2, 4, 8 within each row of 16 lanes, then lane 15 of each row
// added to the next row (rows 1 and 3), then lane 31 to rows 2 and 3.  Lanes with
// no source keep the `old` operand, 0.
__device__ inline int wave_incl_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return x;
}
// One DPP move of a 64-bit value (both halves with the same control).
template <int kCtrl, int kRowMask>
__device__ inline long long dpp_mov64(long long x) {
  const unsigned int lo = static_cast<unsigned int>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(x), kCtrl, kRowMask, 0xF, false));
  const unsigned int hi = static_cast<unsigned int>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(x >> 32), kCtrl, kRowMask, 0xF, false));
  return static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo);
}
// wave_incl_scan for 64-bit values.
__device__ inline long long wave_incl_scan64(long long x) {
  x += dpp_mov64<0x111, 0xF>(x);
  x += dpp_mov64<0x112, 0xF>(x);
  x += dpp_mov64<0x114, 0xF>(x);
  x += dpp_mov64<0x118, 0xF>(x);
  x += dpp_mov64<0x142, 0xA>(x);
  x += dpp_mov64<0x143, 0xC>(x);
  return x;
}

// Wave index as a scalar (the compiler cannot tell that threadIdx.x / 64 is
// uniform across a wave; LDS addresses derived from it must be scalars).
__device__ inline int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }
// Lane index computed afresh where it is used: volatile asm is neither
// hoisted nor merged with an earlier copy, so the values derived from it are
// rebuilt in place instead of being kept (and spilled) across the kernel.
__device__ inline int fresh_lane() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// 16 bytes per lane from global memory straight into LDS
// (global_load_lds_dwordx4): lane l's bytes land at lds + 16 l.  Issued from
// inline asm rather than the builtin: the compiler books the builtin as a flat
// access that may still be pending on the LDS counter, after which it can
// only wait for an LDS read with lgkmcnt(0), i.e. behind every LDS read in
// flight, which defeats reading operands ahead.  The hardware counts these
// loads in vmcnt alone; the kernels wait for them with explicit vmcnt counts,
// and the compiler's own vmcnt waits, not knowing of them, can only come out
// stricter.  (m0 holds the LDS address; one wait state after writing it.)
__device__ inline void lds_dma16(const void* src, FA_LDS void* lds) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane(
      static_cast<unsigned>(reinterpret_cast<__SIZE_TYPE__>(lds)));
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(m0)
               : "memory", "m0");
}

// lds_dma16 with the non-temporal hint (nt): for streams read once per launch,
// whose lines are better not kept in the caches (the GQA decode's K/V tiles).
__device__ inline void lds_dma16_nt(const void* src, FA_LDS void* lds) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane(
      static_cast<unsigned>(reinterpret_cast<__SIZE_TYPE__>(lds)));
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
               :
               : "v"(src), "s"(m0)
               : "memory", "m0");
}

// The same for 4 bytes per lane (global_load_lds_dword): lane l's word lands
// at lds + 4 l.
__device__ inline void lds_dma4(const void* src, FA_LDS void* lds) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane(
      static_cast<unsigned>(reinterpret_cast<__SIZE_TYPE__>(lds)));
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :
               : "v"(src), "s"(m0)
               : "memory", "m0");
}

// LDS transpose read (ds_read_b64_tr_b16).  Within each 16-lane group, result
// lane i, element e comes from source lane 4e + i/4, element i%4: four lanes
// pointing at 4 consecutive dims of token row e give every lane one dim of 4
// consecutive tokens (see the V^T operand addressing in the kernel).
__device__ inline bf16x4 lds_read_tr4(const unsigned char* p) {
  typedef short shortx4 __attribute__((ext_vector_type(4)));
  shortx4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((FA_LDS shortx4*)(p));
  return __builtin_bit_cast(bf16x4, v);
}

// Values that are uniform but may have been computed in vector registers are
// moved to scalars before they form a buffer resource (a vector resource
// would need a loop over lanes).
__device__ inline int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ inline const unsigned char* uniform(const unsigned char* p) {
  const unsigned long long v = reinterpret_cast<unsigned long long>(p);
  const unsigned int lo = __builtin_amdgcn_readfirstlane(static_cast<unsigned int>(v));
  const unsigned int hi = __builtin_amdgcn_readfirstlane(static_cast<unsigned int>(v >> 32));
  return reinterpret_cast<const unsigned char*>((static_cast<unsigned long long>(hi) << 32) | lo);
}

// Max / sum with the lane 16 (32) positions away: gfx950 lane-swap VALU ops
// (v_permlane16_swap / v_permlane32_swap on two copies of x leave the two
// partners' values in the two outputs), no LDS traffic.  The outputs are
// copied to scalars before reinterpretation: a bit cast taken directly on a
// vector element reads element 0 with this compiler.
__device__ inline floatx2 swap16(float x) {
  const unsigned u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const unsigned r0 = r[0], r1 = r[1];
  floatx2 o;
  o[0] = __uint_as_float(r0);
  o[1] = __uint_as_float(r1);
  return o;
}
__device__ inline floatx2 swap32(float x) {
  const unsigned u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const unsigned r0 = r[0], r1 = r[1];
  floatx2 o;
  o[0] = __uint_as_float(r0);
  o[1] = __uint_as_float(r1);
  return o;
}
__device__ inline float max_xor16(float x) {
  const floatx2 v = swap16(x);
  return fmaxf(v[0], v[1]);
}
__device__ inline float max_xor32(float x) {
  const floatx2 v = swap32(x);
  return fmaxf(v[0], v[1]);
}
__device__ inline float sum_xor16(float x) {
  const floatx2 v = swap16(x);
  return v[0] + v[1];
}
__device__ inline float sum_xor32(float x) {
  const floatx2 v = swap32(x);
  return v[0] + v[1];
}

template <int V>
struct IntTag {
  static constexpr int value = V;
};

// f(IntTag<0>{}), ..., f(IntTag<N-1>{}): an unrolled loop whose index is a
// compile-time constant (needed for instruction immediates).
template <typename F, int... Is>
__device__ inline void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(IntTag<Is>{}), ...);
}
template <int N, typename F>
__device__ inline void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

}  // namespace fa
