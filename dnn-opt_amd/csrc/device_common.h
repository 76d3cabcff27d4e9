// device_common.h -- helpers shared by the gfx950 kernels.
//
// Everything here is device code for CDNA4 (wave64).  Buffer loads go through
// a buffer resource descriptor so that reads past the end of an operand return
// zero instead of faulting: that is how ragged tails (prime N, K not a multiple
// of the unroll) are handled without padded copies.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dnnopt_dev {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Word 3 of a raw (untyped, stride 0) buffer descriptor on gfx9-class parts:
// 32-bit data format, no swizzle.  Offsets >= num_records read as zero.
constexpr int kRsrcWord3 = 0x00020000;

// Offset used to force an out-of-range (zero-returning) buffer read.
constexpr uint32_t kOobOffset = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             kRsrcWord3);
}

__device__ __forceinline__ u32x4 buf_load_x4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

__device__ __forceinline__ uint32_t buf_load_x1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

__device__ __forceinline__ uint16_t buf_load_u16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

__device__ __forceinline__ float as_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ uint32_t as_u32(float f) { return __builtin_bit_cast(uint32_t, f); }

// bf16 bits -> fp32 (exact).
__device__ __forceinline__ float bf16_lo(uint32_t packed) { return as_f32(packed << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t packed) { return as_f32(packed & 0xFFFF0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return as_f32((uint32_t)b << 16); }

// fp32 -> bf16 with round to nearest, ties to even on the low 16 bits, and no
// NaN special case: the integer formula of the reference's bfloat16_t
// (include/dnnopt/gemm/gemm_types.h:18-24).  Returns the rounded value as fp32.
__device__ __forceinline__ float round_bf16(float f) {
    uint32_t u = as_u32(f);
    u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
    return as_f32(u);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = as_u32(f);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// Wave index as a scalar (lets the compiler keep per-wave addresses in SGPRs).
__device__ __forceinline__ int wave_id() {
    return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}
__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63); }

// Reference epilogue of the fp32 kernels: beta == 0 -> alpha*acc (C unread),
// otherwise fma(alpha, acc, beta*C)  (gemm_tiny_fp32.cpp:200-207,
// gemm_smallm_wide_fp32.cpp:47-59).
__device__ __forceinline__ float epilogue(float acc, float alpha, float beta, const float* c) {
    if (beta == 0.0f) return alpha * acc;
    return __builtin_fmaf(alpha, acc, beta * (*c));
}

// Cross-workgroup ticket: every workgroup of a split-K group calls this after
// its partial results are stored.  Returns true in exactly one workgroup -- the
// last to arrive -- after which that workgroup may read every partial.  The
// release fence before the atomic makes this workgroup's partial stores
// visible at device (agent) scope, across XCD L2s; the acquire fence in the
// last workgroup makes the other workgroups' stores visible to it.  The last
// workgroup resets the ticket so the next launch starts from zero.
__device__ __forceinline__ bool split_ticket(unsigned* ticket, unsigned nsplits, int* lds_flag) {
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned t = atomicAdd(ticket, 1u);
        bool last = (t == nsplits - 1);
        // Every other workgroup of the group has already taken its ticket.
        if (last) atomicExch(ticket, 0u);
        *lds_flag = last ? 1 : 0;
    }
    __syncthreads();
    bool last = *lds_flag != 0;
    if (last) __threadfence();
    return last;
}

}  // namespace dnnopt_dev
