// Shared device helpers for the gfx950 W4A16 qlinear / routed-MoE kernels.
//
// Conventions used by every kernel in this library:
//   * wave64; lane = threadIdx.x & 63.
//   * v_mfma_f32_16x16x32_bf16 operand layout: lane l supplies row (l & 15) of
//     A and column (l & 15) of B, each with 8 k-values from k-octet (l >> 4);
//     the 4 fp32 results of lane l are D[4*(l>>4) + e][l & 15], e = 0..3.
//   * Packed int4 weights are the portable K-packed format: uint8 [N][K/2],
//     even k in the low nibble, signed two's complement.  One 32-bit word holds
//     8 consecutive k.  dequant8() turns it into four bf16 pairs
//     (k0,k4) (k1,k5) (k2,k6) (k3,k7), each value being 136 + q.
//   * Activations feeding a W4 MFMA are therefore stored "octet-interleaved":
//     within each block of 8 k the order is k0 k4 k1 k5 k2 k6 k3 k7, so one
//     16-byte load gives the matching A operand.  The +136 offset is removed
//     per group with the precomputed term -136 * sum_group(x) ("xneg").
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dflash {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kNibbleMask = 0x000F000Fu;
constexpr uint32_t kBf16Magic = 0x43004300u;   // bf16 pair (128.0, 128.0)
constexpr float kDequantOffset = 136.0f;       // 128 + 8 (sign flip of the nibble)

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt untouched).  Used right after loads
// issued under a condition inside a loop, so later uses of those registers
// need no conservative full wait on every iteration.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Workgroup barrier for LDS traffic only: waits for this wave's LDS operations
// (lgkmcnt(0)) but not for its vector-memory loads still in flight.
// __syncthreads() waits for whatever loads the compiler's counter tracking still
// sees (often vmcnt(0), a prefetch pipeline's worth of outstanding global loads),
// but direct-to-LDS loads issued in an earlier iteration of a loop can be
// invisible to it: it may then be a bare s_barrier.  The empty asm statements keep the
// compiler from moving memory accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left at their maxima
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Load of a wave-uniform element through the constant address space: with a
// readfirstlane'd index it becomes s_load (counted by lgkmcnt), so it never
// waits behind the vector loads a wave keeps in flight.  Only for memory the
// running kernel does not write.
template <typename T>
__device__ __forceinline__ T ld_const(const T* p, int i) {
  i = __builtin_amdgcn_readfirstlane(i);
  return ((const __attribute__((address_space(4))) T*)(p))[i];  // address-space cast
}

typedef int i32x4 __attribute__((ext_vector_type(4)));

// 16-byte wave-uniform record as one s_load_dwordx4.
__device__ __forceinline__ int4 ld_const_int4(const int4* p, int i) {
  i = __builtin_amdgcn_readfirstlane(i);
  const i32x4 v = ((const __attribute__((address_space(4))) i32x4*)(p))[i];
  return make_int4(v.x, v.y, v.z, v.w);
}

// Raw buffer resource over [base, base + bytes): loads through it take a 32-bit
// VGPR byte offset plus a wave-uniform SGPR offset, and read 0 past the end.
typedef __amdgpu_buffer_rsrc_t buf_rsrc;
constexpr int kBufferDword3 = 0x00020000;  // 32-bit data format, raw (stride 0) addressing

__device__ __forceinline__ buf_rsrc make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                           kBufferDword3);
}
__device__ __forceinline__ uint4 buf_load16(buf_rsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff),
                                                                         static_cast<int>(soff), 0));
}
__device__ __forceinline__ float buf_load_f32(buf_rsrc r, uint32_t voff, uint32_t soff) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(voff), static_cast<int>(soff), 0));
}

__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t bits) {
  uint32_t d;
  // gfx9 VOP3 reads at most one SGPR: mask from an SGPR, the magic bits from a VGPR.
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "s"(mask), "v"(bits));
  return d;
}

// 8 signed nibbles -> 4 bf16 pairs holding 136+q in the octet-interleaved order.
__device__ __forceinline__ uint4 dequant8(uint32_t w) {
  w ^= 0x88888888u;
  uint4 r;
  r.x = and_or(w, kNibbleMask, kBf16Magic);
  r.y = and_or(w >> 4, kNibbleMask, kBf16Magic);
  r.z = and_or(w >> 8, kNibbleMask, kBf16Magic);
  r.w = and_or(w >> 12, kNibbleMask, kBf16Magic);
  return r;
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ f32x4 mfma16x16x32(uint4 a, uint4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma16x16x4f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN stays NaN): one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Raw scale bits (no conversion at load time, so a prefetched scale does not
// force a wait on the loads issued before it) and their fp32 value.
__device__ __forceinline__ uint32_t load_scale_bits(const uint16_t* p) { return *p; }
__device__ __forceinline__ uint32_t load_scale_bits(const float* p) { return __float_as_uint(*p); }
template <typename ScaleT>
__device__ __forceinline__ float scale_value(uint32_t bits) {
  return sizeof(ScaleT) == 2 ? __uint_as_float(bits << 16) : __uint_as_float(bits);
}

template <typename ScaleT>
__device__ __forceinline__ float load_scale(const ScaleT* p);
template <>
__device__ __forceinline__ float load_scale<uint16_t>(const uint16_t* p) { return bf16_to_f32(*p); }
template <>
__device__ __forceinline__ float load_scale<float>(const float* p) { return *p; }

// Lane quarters <-> words: word D of lane quarter Q becomes word Q of lane quarter D (a 4 x 4
// transpose of four 32-bit words across the wave's four 16-lane quarters).  permlane32_swap
// exchanges the upper 32 lanes of its first operand with the lower 32 of its second,
// permlane16_swap the odd 16-lane rows of the first with the even rows of the second.
__device__ __forceinline__ void quarter_transpose(uint32_t (&w)[4]) {
  auto s02 = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
  auto s13 = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
  auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
  auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
  w[0] = s01[0];
  w[1] = s01[1];
  w[2] = s23[0];
  w[3] = s23[1];
}

// Interleaved position of column c inside its octet (k0 k4 k1 k5 k2 k6 k3 k7).
__device__ __forceinline__ int octet_slot(int c) { return (c & ~7) | ((c & 3) << 1) | ((c >> 2) & 1); }

// Sum over the 16 lanes that share (lane >> 4): DPP row rotations, no LDS trip.
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f32<0x121>(v);  // row_ror:1
  v += dpp_f32<0x122>(v);  // row_ror:2
  v += dpp_f32<0x124>(v);  // row_ror:4
  v += dpp_f32<0x128>(v);  // row_ror:8
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// g * sigmoid(g); the product is rounded to bf16 afterwards, so the 1-ulp reciprocal suffices.
__device__ __forceinline__ float silu(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

}  // namespace dflash
