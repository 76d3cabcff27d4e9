// k_wide.hip -- last-resort GEMM for operands the tiled kernels cannot
// address (gfx950).
//
// Every other kernel of this library reads through buffer descriptors with
// 32-bit offsets from the start of a workgroup's tile, so a tile whose rows
// span more than 2^31 bytes (a K x M A with a long k, a B stored N x K whose
// rows are gigabytes, k in the tens of millions with row-major A) is refused
// by their planners.  The reference computes such shapes (plain pointers on
// the CPU), so they land here: 64-bit addressing, any layout, every data
// type of the path, speed secondary.
//
// One workgroup of 16 waves computes 64 consecutive outputs of one row of C
// (lane = column).  Wave w sums its contiguous k-range [w K / 16, (w + 1) K /
// 16) in ascending k; the 16 wave sums are added in wave order through LDS,
// so the result is the same on every call.  fp32 modes accumulate with fused
// multiply-adds and finish with the fp32 kernels' epilogue (and bias); int8
// accumulates exactly in int32 and stores int32, or the per-column scaled /
// dynamically dequantized fp32 C of the int8 kernels.
#include <type_traits>

#include "device_common.h"
#include "kernels.h"

using namespace dnnopt_dev;

namespace dnnopt_hip {

namespace {

constexpr int kWideWaves = 16;

template <int MODE>
__device__ __forceinline__ float wide_val(const void* p, long long idx) {
    if constexpr (MODE == kWideBF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[idx]);
    else if constexpr (MODE == kWideF2B) return round_bf16(static_cast<const float*>(p)[idx]);
    else return static_cast<const float*>(p)[idx];
}

}  // namespace

template <int MODE, int TA, int TB>
__global__ __launch_bounds__(kWideWaves * 64) void dnnopt_wide(WideArgs p) {
    using Acc = typename std::conditional<MODE == kWideS8, int32_t, float>::type;
    __shared__ Acc red[kWideWaves][64];
    const int lane = lane_id(), w = wave_id();
    const long long tn = (p.N + 63) / 64;
    const long long blk = (long long)blockIdx.y * gridDim.x + blockIdx.x;
    if (blk >= tn * p.M) return;  // whole workgroup
    const long long i = blk / tn;
    const long long j = (blk % tn) * 64 + lane;
    const bool ok = j < p.N;
    const long long k0 = (long long)p.K * w / kWideWaves, k1 = (long long)p.K * (w + 1) / kWideWaves;
    // A(i, k) at a_base + k * a_step, B(k, j) at b_base + k * b_step.
    const long long a_base = TA ? i : i * p.lda, a_step = TA ? p.lda : 1;
    const long long b_base = TB ? j * p.ldb : j, b_step = TB ? 1 : p.ldb;
    Acc acc = 0;
    if (ok) {
#pragma unroll 4
        for (long long k = k0; k < k1; ++k) {
            if constexpr (MODE == kWideS8) {
                acc += (int32_t) static_cast<const int8_t*>(p.A)[a_base + k * a_step] *
                       (int32_t) static_cast<const int8_t*>(p.B)[b_base + k * b_step];
            } else {
                acc = __builtin_fmaf(wide_val<MODE>(p.A, a_base + k * a_step),
                                     wide_val<MODE>(p.B, b_base + k * b_step), acc);
            }
        }
    }
    red[w][lane] = acc;
    __syncthreads();
    if (w != 0 || !ok) return;
    Acc sum = red[0][lane];
#pragma unroll
    for (int v = 1; v < kWideWaves; ++v) sum += red[v][lane];
    const long long off = i * p.ldc + j;
    if constexpr (MODE == kWideS8) {
        if (p.epi == 0) {
            static_cast<int32_t*>(p.C)[off] = sum;
        } else {
            float* c = static_cast<float*>(p.C) + off;
            const float dq = p.amax ? dyn_dequant_scale(p.amax, p.alpha) : 0.0f;
            *c = s8_out(sum, (int)j, p.scale, p.amax, dq, p.beta, c);
        }
    } else {
        float* c = static_cast<float*>(p.C) + off;
        *c = add_bias(epilogue(sum, p.alpha, p.beta, c), p.bias, (int)j);
    }
}

template <int MODE>
static hipError_t launch_wide_mode(const WideArgs& a, dim3 grid, hipStream_t s) {
    const dim3 blk(kWideWaves * 64);
    if (!a.transA && !a.transB) hipLaunchKernelGGL((dnnopt_wide<MODE, 0, 0>), grid, blk, 0, s, a);
    else if (a.transA && !a.transB) hipLaunchKernelGGL((dnnopt_wide<MODE, 1, 0>), grid, blk, 0, s, a);
    else if (!a.transA && a.transB) hipLaunchKernelGGL((dnnopt_wide<MODE, 0, 1>), grid, blk, 0, s, a);
    else hipLaunchKernelGGL((dnnopt_wide<MODE, 1, 1>), grid, blk, 0, s, a);
    return hipGetLastError();
}

dim3 wide_grid(int M, int N) {
    const long long blocks = (long long)M * ((N + 63) / 64);
    const long long gx = blocks < (1ll << 30) ? blocks : (1ll << 30);
    return dim3((unsigned)gx, (unsigned)((blocks + gx - 1) / gx), 1);
}

int wide_threads() { return kWideWaves * 64; }

hipError_t launch_wide(int mode, const WideArgs& a, hipStream_t s) {
    if (a.M <= 0 || a.N <= 0) return hipSuccess;
    const dim3 grid = wide_grid(a.M, a.N);
    switch (mode) {
        case kWideF32: return launch_wide_mode<kWideF32>(a, grid, s);
        case kWideBF16: return launch_wide_mode<kWideBF16>(a, grid, s);
        case kWideF2B: return launch_wide_mode<kWideF2B>(a, grid, s);
        case kWideS8: return launch_wide_mode<kWideS8>(a, grid, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace dnnopt_hip
