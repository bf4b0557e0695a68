// LDS staging and MFMA operand helpers shared by the attention kernels
// (forward in attention.hip, backward in attention_bwd.hip).
//
// Register layouts of v_mfma_f32_32x32x16_bf16 (lane l, g = l / 32, c = l % 32):
//   A operand: row c, 8 consecutive k-slots of half g
//   B operand: col c, 8 consecutive k-slots of half g
//   C/D:       reg r holds row 8*(r/4) + 4*g + (r%4), col c
#pragma once

#include "mk_common.h"

namespace mk {
namespace attn {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;
typedef int i32x4_t __attribute__((ext_vector_type(4)));

constexpr int kBufferWord3 = 0x00020000;  // raw buffer descriptor, gfx9 family

template <bool B>
struct Flag {
  static constexpr bool value = B;
};
template <int N>
struct Int {
  static constexpr int value = N;
};

__device__ inline bf16x8_t as_bf16x8(const u32x4_t& v) {
  bf16x8_t r;
  __builtin_memcpy(&r, &v, 16);
  return r;
}

// 8 fp32 -> 8 bf16 (RNE, v_cvt_pk_bf16_f32) as one 8-slot MFMA operand
__device__ inline bf16x8_t pack8(float a0, float a1, float a2, float a3, float a4, float a5, float a6, float a7) {
  const f32x2_t v0 = {a0, a1}, v1 = {a2, a3}, v2 = {a4, a5}, v3 = {a6, a7};
  const u32x4_t w = {__builtin_bit_cast(uint32_t, __builtin_convertvector(v0, bf16x2_t)),
                     __builtin_bit_cast(uint32_t, __builtin_convertvector(v1, bf16x2_t)),
                     __builtin_bit_cast(uint32_t, __builtin_convertvector(v2, bf16x2_t)),
                     __builtin_bit_cast(uint32_t, __builtin_convertvector(v3, bf16x2_t))};
  return as_bf16x8(w);
}

// raw buffer descriptor over [base, base + bytes): loads past the end return
// zeros (word1: base bits 47:32, stride 0; word2: size; word3: gfx9 format)
__device__ inline i32x4_t tile_desc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return i32x4_t{int(uint32_t(a)), int(uint32_t(a >> 32) & 0xFFFFu), int(bytes), kBufferWord3};
}

// LDS byte address of a __shared__ location: the low 32 bits of its generic
// address (the shared aperture base has zero low bits).  Taking them directly
// avoids the address-space cast's null check, which keeps 64-bit generic
// addresses alive in SGPRs.
__device__ inline uint32_t lds_addr(const void* p) {
  return uint32_t(reinterpret_cast<uintptr_t>(p));
}

// One 1 KB copy HBM/L2 -> LDS: lane l loads 16 bytes at byte offset voff of
// the descriptor's range and the buffer unit writes them to LDS bytes
// [dst + 16 l, dst + 16 l + 16).  Issued from inline assembly so that the
// compiler does not track it: it inserts no vmcnt wait of its own for these
// copies, and the kernel waits for them explicitly (wait_copies) before the
// barrier that hands the data to the other waves.  M0 holds the LDS address
// (set by the compiler from the constraint).
// The descriptor and the LDS address pass through readfirstlane here, at the
// operand, so they are in SGPRs however the caller computed them.  A VALU
// write of an SGPR (v_readfirstlane) needs 5 wait states before a VMEM
// instruction reads that SGPR, and the compiler's hazard pass does not look
// inside inline assembly, so the copy is preceded by s_nop 4 (5 wait states;
// this also covers the one the M0 write needs).  Without it a descriptor
// word written just before the copy can be read stale.
__device__ inline void copy_to_lds(const i32x4_t& rsrc, uint32_t dst, int voff) {
  const i32x4_t r = {__builtin_amdgcn_readfirstlane(rsrc.x), __builtin_amdgcn_readfirstlane(rsrc.y),
                     __builtin_amdgcn_readfirstlane(rsrc.z), __builtin_amdgcn_readfirstlane(rsrc.w)};
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(r), "{m0}"(__builtin_amdgcn_readfirstlane(dst))
               : "memory");
}

// copy_to_lds with an SGPR byte offset added to voff (the same wave-uniform
// step for every lane), for callers whose descriptor and offset are
// wave-uniform values the compiler keeps in SGPRs (computed by SALU, not
// passed through a VALU readfirstlane right before the copy): it waits only
// the one state the M0 write needs (s_nop 0).  tests/test_asm_hazards.py
// checks every copy of the compiled kernels for a VALU write of one of its
// SGPRs fewer than 5 wait states earlier.
__device__ inline void copy_to_lds_so(const i32x4_t& rsrc, uint32_t dst, int voff, uint32_t soff) {
  const i32x4_t r = {__builtin_amdgcn_readfirstlane(rsrc.x), __builtin_amdgcn_readfirstlane(rsrc.y),
                     __builtin_amdgcn_readfirstlane(rsrc.z), __builtin_amdgcn_readfirstlane(rsrc.w)};
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(r), "s"(__builtin_amdgcn_readfirstlane(soff)),
                 "{m0}"(__builtin_amdgcn_readfirstlane(dst))
               : "memory");
}

// wait until every copy this wave has issued has landed in LDS
__device__ inline void wait_copies() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// workgroup barrier ordering LDS accesses only (waits for lgkmcnt, not vmcnt)
__device__ inline void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// 4 bf16 of one LDS column block (ds_read_b64_tr_b16), as two 32-bit words:
// the 16 lanes of a group address a 4-row x 16-column block (4 lanes per row,
// 8 bytes each) and lane i of the group receives column i of it.
__device__ inline uint2 lds_read_tr(const uint16_t* p) {
  const i16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p));
  return __builtin_bit_cast(uint2, v);
}

// Values of lanes l and l ^ 32 in one VALU op, without the LDS path of
// ds_bpermute: v_permlane32_swap on two copies of v leaves v[l % 32] in the
// first result and v[l % 32 + 32] in the second, in every lane.  The empty
// asm keeps the optimiser from treating the two operands as one value.
__device__ inline void lane_halves(float v, float& lo, float& hi) {
  const uint32_t a = __builtin_bit_cast(uint32_t, v);
  uint32_t b = a;
  asm volatile("" : "+v"(b));
  const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
  lo = __builtin_bit_cast(float, static_cast<uint32_t>(r[0]));
  hi = __builtin_bit_cast(float, static_cast<uint32_t>(r[1]));
}

// lane_halves without the asm: an inline asm statement ends the compiler's
// scheduling region, which would keep independent MFMAs from being
// interleaved across it.  The register allocator gives the two tied operands
// of v_permlane32_swap separate registers (a copy) by itself.
__device__ inline void lane_halves_sched(float v, float& lo, float& hi) {
  const uint32_t a = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane32_swap(a, a, false, false);
  lo = __builtin_bit_cast(float, static_cast<uint32_t>(r[0]));
  hi = __builtin_bit_cast(float, static_cast<uint32_t>(r[1]));
}

}  // namespace attn
}  // namespace mk
