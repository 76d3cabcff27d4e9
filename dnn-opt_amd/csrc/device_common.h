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

// Buffer range in bytes, clamped to 2^31 - 1.  Written as a plain select:
// the HIP min() template for 64-bit values is not recognised as wave-uniform,
// which turns every load through the descriptor into a readfirstlane loop.
__device__ __forceinline__ uint32_t range31(size_t bytes) {
    return bytes > 0x7FFFFFFFull ? 0x7FFFFFFFu : (uint32_t)bytes;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             kRsrcWord3);
}

__device__ __forceinline__ u32x4 buf_load_x4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// Cache-policy operand of the buffer intrinsics on gfx950: bit 0 = sc0,
// bit 1 = nt, bit 4 = sc1.  sc0|sc1 is system scope: loads miss in every
// cache level and stores write through to memory, which makes data written by
// one workgroup visible to another on any XCD without an L2 writeback or
// invalidate.  nt marks streaming data that is used once.
constexpr int kAuxNT = 2;
constexpr int kAuxCoherent = 17;

__device__ __forceinline__ u32x4 buf_load_x4_stream(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kAuxNT));
}

__device__ __forceinline__ f32x4 buf_load_x4_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kAuxCoherent));
}

__device__ __forceinline__ void buf_store_x4(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, 0);
}

__device__ __forceinline__ void buf_store_x4_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, kAuxCoherent);
}

__device__ __forceinline__ uint32_t buf_load_x1_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kAuxCoherent);
}

__device__ __forceinline__ void buf_store_x1(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t v) {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, 0);
}

__device__ __forceinline__ void buf_store_x1_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t v) {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, kAuxCoherent);
}

__device__ __forceinline__ uint32_t buf_load_x1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

__device__ __forceinline__ uint16_t buf_load_u16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// Dword buffer loads ignore the two low address bits, so 16 bytes that do not
// start on a 4-byte boundary (rows of an odd-length bf16 or int8 matrix) are
// read as the enclosing aligned 20 bytes and funnel-shifted into place.  The
// descriptor must start on a 4-byte boundary (see rsrc_aligned) and `off` is
// the byte offset from it; shift 0 returns the aligned load unchanged.
__device__ __forceinline__ u32x4 buf_load_x4_unaligned(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const uint32_t sh = off & 3u;
    const uint32_t o = off - sh;
    const u32x4 v = buf_load_x4(r, o);
    const uint32_t e = buf_load_x1(r, o + 16u);
    u32x4 out;
    out[0] = __builtin_amdgcn_alignbyte(v[1], v[0], sh);
    out[1] = __builtin_amdgcn_alignbyte(v[2], v[1], sh);
    out[2] = __builtin_amdgcn_alignbyte(v[3], v[2], sh);
    out[3] = __builtin_amdgcn_alignbyte(e, v[3], sh);
    return out;
}

// Descriptor for `bytes` bytes starting at `base`, with the start rounded
// down to 4 bytes; *lo receives the bytes skipped (add it to every offset).
// The range check of a dword load rejects a dword that extends past the
// range, so the range is also rounded up to whole dwords: the extra bytes lie
// in the same aligned dword (and page) as the last valid byte, and every
// kernel masks or discards what it reads there.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_aligned(const void* base, size_t bytes, uint32_t* lo) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(base);
    *lo = (uint32_t)(a & 3u);
    const size_t total = (bytes + *lo + 3u) & ~(size_t)3u;
    return make_rsrc(reinterpret_cast<const void*>(a - *lo), total > 0x7FFFFFFFull ? 0x7FFFFFFFu : (uint32_t)total);
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

// Balanced split-k decomposition: workgroup g of G over T column tiles
// (G >= T).  The first G % T tiles get G/T + 1 k-splits, the others G/T, and
// workgroups are numbered tile by tile.
struct SplitPos {
    int tile, split, nsplit;
};

__host__ __device__ __forceinline__ SplitPos split_pos(int g, int G, int T) {
    const int q = G / T, r = G % T;
    const int big = r * (q + 1);
    if (g < big) return SplitPos{g / (q + 1), g % (q + 1), q + 1};
    const int h = g - big;
    return SplitPos{r + h / q, h % q, q};
}

__host__ __device__ __forceinline__ int splits_of_tile(int t, int G, int T) {
    return G / T + (t < G % T ? 1 : 0);
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

// Per-column bias added to a finished output as its own rounding (nothing
// when bias is null): the oneDNN hook adds its bias to the completed C
// (integration/onednn/0001-dnnopt-integration.patch:355-362).
//
// add_rn / mul_rn round on their own: contraction is off inside them, so the
// compiler cannot fuse them with a product or sum computed before (a plain
// a + b after y = alpha * acc may otherwise become one fma).
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}
__device__ __forceinline__ float add_bias(float y, const float* bias, int n) {
    return bias ? add_rn(y, bias[n]) : y;
}

// Per-tensor int8 quantization scale of the fp32-API gemm_int8: max|X| / 127,
// or 1 when the tensor is all zero (src/gemm/gemm_driver_generic.cpp:49-67).
// `amax_bits` is the bit pattern of max|X|.
__device__ __forceinline__ float quant_scale_bits(uint32_t amax_bits) {
    const float amax = as_f32(amax_bits);
    return amax == 0.0f ? 1.0f : amax / 127.0f;
}

// Dynamic int8 quantization of one value (fp32-API gemm_int8,
// src/gemm/gemm_pack_int8.cpp:29-71): q = clamp(rint(x * inv), -128, 127) as
// an int.  The conversion of NaN gives 0 and large values saturate before the
// clamp, so the result equals the clamp-then-convert form for every input.
__device__ __forceinline__ int quant_s8(float x, float inv) {
    const int v = (int)__builtin_rintf(x * inv);
    return v > 127 ? 127 : (v < -128 ? -128 : v);
}

// Quantization of the fp32-API gemm_int8 at M <= 8, the reference's small-M
// route (src/gemm/gemm_smallm_int8.cpp:151, 159, 233, 280-281): a true
// division, q = clamp(rint(x / s), -128, 127).  With inv = 1 / s correctly
// rounded, q0 = x * inv is within an ulp of x / s, the residual
// r = fma(-q0, s, x) is exact, and fma(r, inv, q0) is the correctly rounded
// quotient whenever nothing underflows (Markstein's theorem).  For scales in
// [2^-64, 2^64] every quotient near a half-integer -- the only ones where the
// rounding to an integer can change -- is far from underflow; quotients that
// do underflow are below 0.5 and round to 0 either way.  Scales outside that
// range take the compiler's correctly rounded division (QuantDiv::exact).
struct QuantDiv {
    float s, inv;
    bool exact;
};
__device__ __forceinline__ QuantDiv quant_div_of(uint32_t amax_bits) {
    const float s = quant_scale_bits(amax_bits);
    const bool in_range = s >= 0x1p-64f && s <= 0x1p64f;
    return QuantDiv{s, 1.0f / s, !in_range};
}
// CLAMP = false when |x| <= max|X| is known: then |x / s| <= 127 (1 + 2^-23)
// and the rounded value lies in [-127, 127] already (NaN converts to 0).
template <bool EXACT, bool CLAMP>
__device__ __forceinline__ int quant_s8_div(float x, const QuantDiv& d) {
    float q;
    if constexpr (EXACT) {
        q = x / d.s;
    } else {
        const float q0 = x * d.inv;
        q = __builtin_fmaf(__builtin_fmaf(-q0, d.s, x), d.inv, q0);
    }
    const int v = (int)__builtin_rintf(q);
    if constexpr (!CLAMP) return v;
    return v > 127 ? 127 : (v < -128 ? -128 : v);
}

// Output of the fp32-API gemm_int8 at M <= 8 (t = alpha * (sA * sB)):
//   M == 1 (gemm_mx1_int8, src/gemm/gemm_smallm_int8.cpp:170-175):
//     beta == 0 ? t * acc : fma(beta, C, t * acc) -- the reference's
//     `result + beta * C[j]` contracts only the beta * C product, since
//     `result` also feeds the beta == 0 store;
//   M >= 2 (gemm_smallm_int8_smmla, :243-250, :356-383): C is first set to 0
//     or beta * C, then C + t * acc is stored -- two roundings.
// C is read only when beta != 0 (c_old holds it then).
__device__ __forceinline__ float smallm_out(int32_t acc, bool one_row, float t, float beta, float c_old) {
    const float r = mul_rn(t, (float)acc);
    if (one_row) return beta == 0.0f ? r : __builtin_fmaf(beta, c_old, r);
    const float c0 = beta == 0.0f ? 0.0f : (beta == 1.0f ? c_old : mul_rn(c_old, beta));
    return add_rn(c0, r);
}

// The maxima of A (part[0, ga)) and B (part[ga, ga + gb)), ga + gb <= 1024,
// reduced by one wave on its own (no barrier): 16 consecutive partials per
// lane, read as four 16-byte loads.  The buffer range is rounded up to whole
// 16-byte loads (the partials' allocation is padded to 256 bytes); values
// past ga + gb are masked.
__device__ __forceinline__ void wave_maxima(const unsigned* part, int ga, int gb, unsigned* ma, unsigned* mb) {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(part, ((uint32_t)(ga + gb) * 4u + 15u) & ~15u);
    const int lane = lane_id();
    u32x4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = buf_load_x4(r, (uint32_t)(lane * 16 + 4 * j) * 4u);
    unsigned a = 0, b = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = lane * 16 + 4 * j + e;
            if (i < ga) a = v[j][e] > a ? v[j][e] : a;
            else if (i < ga + gb) b = v[j][e] > b ? v[j][e] : b;
        }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned oa = (unsigned)__shfl_xor((int)a, off, 64), ob = (unsigned)__shfl_xor((int)b, off, 64);
        a = oa > a ? oa : a;
        b = ob > b ? ob : b;
    }
    *ma = a;
    *mb = b;
}

// fp32 output of an exact int32 accumulator (EPI 1 of the int8 kernels):
//   amax == nullptr: per-column dequantization, (float)acc * scale[n];
//   amax != nullptr: the dynamic per-tensor dequantization of the fp32-API
//     gemm_int8, with dq = (sA * sB) * alpha from dyn_dequant_scale():
//     beta == 0 ? dq * acc : fma(dq, acc, beta * C)
//     (src/gemm/gemm_ukernel_int8_neon.cpp:87-131).
// Every product and the conversion round once, as in the reference.
__device__ __forceinline__ float dyn_dequant_scale(const unsigned* amax, float alpha) {
    return mul_rn(mul_rn(quant_scale_bits(amax[0]), quant_scale_bits(amax[1])), alpha);
}
__device__ __forceinline__ float s8_out(int32_t acc, int n, const float* scale, const unsigned* amax, float dq,
                                        float beta, const float* c) {
    if (!amax) return mul_rn((float)acc, scale[n]);
    if (beta == 0.0f) return mul_rn(dq, (float)acc);
    return __builtin_fmaf(dq, (float)acc, mul_rn(beta, *c));
}

// Cross-workgroup ticket: every workgroup of a split-k group calls this after
// storing its partial sums with coherent (sc0 sc1, write-through) stores.
// Returns true in exactly one workgroup -- the last to arrive -- which then
// reads every partial with coherent loads.
//
// Protocol: each wave waits until its own stores have completed (vmcnt(0):
// a write-through store completes once memory holds it); the barrier then
// puts all of them before thread 0's atomic increment, which is performed at
// memory (system scope).  The workgroup that draws the last ticket reads the
// partials only after observing it, with loads that bypass every cache.  No
// agent-scope fence is used: on gfx950 those are whole-L2 writebacks and
// invalidates.  The last workgroup resets the ticket for the next launch.
__device__ __forceinline__ bool split_ticket(unsigned* ticket, unsigned nsplits, int* lds_flag) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's stores are in memory
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned t = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        const bool last = (t == nsplits - 1);
        // Every other workgroup of the group has already taken its ticket.
        if (last) __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        *lds_flag = last ? 1 : 0;
    }
    __syncthreads();
    return *lds_flag != 0;
}

// One 16-byte-per-lane buffer load into LDS: lane l's bytes land at
// lds + 16 l (lds wave-uniform).  The builtin exists only for the device
// pass; the host pass never runs the kernel body.
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, char* lds, uint32_t voffset) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voffset, 0, 0, 0);
#else
    (void)r;
    (void)lds;
    (void)voffset;
#endif
}

// As lds_dma16, for data read once (non-temporal, kAuxNT).
__device__ __forceinline__ void lds_dma16_stream(__amdgpu_buffer_rsrc_t r, char* lds, uint32_t voffset) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voffset, 0, 0,
                                             kAuxNT);
#else
    (void)r;
    (void)lds;
    (void)voffset;
#endif
}

// s_waitcnt vmcnt(n) (n < 64), other counters not waited on.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

}  // namespace dnnopt_dev
