#pragma once
/// @file gemm_types.h
/// Value types shared by the GEMM entry points.
///
/// Layout contract (reference: include/dnnopt/gemm/gemm_types.h:11-39 for
/// bfloat16_t, :203-219 for GemmAlgo): bfloat16_t is a 2-byte POD holding the
/// upper 16 bits of an IEEE-754 binary32 value, and GemmAlgo keeps the same
/// enumerator order so values passed across the ABI keep their meaning.
///
/// The FP8 storage types of the reference (gemm_types.h:41-199) are not part of
/// the small/irregular GEMM path and are not declared here.

#include <cstdint>
#include <cstring>

namespace dnnopt {

/// bfloat16 storage: sign, 8 exponent bits, 7 mantissa bits.
struct bfloat16_t {
    uint16_t raw_bits;

    bfloat16_t() = default;
    constexpr explicit bfloat16_t(uint16_t raw, bool) : raw_bits(raw) {}

    /// Narrow a float with round-to-nearest, ties to even on the dropped
    /// 16 bits.  Like the reference (gemm_types.h:18-24) there is no special
    /// case for NaN: the rounding increment is applied to every bit pattern.
    explicit bfloat16_t(float f) {
        uint32_t bits;
        std::memcpy(&bits, &f, sizeof bits);
        const uint32_t lsb = (bits >> 16) & 1u;
        raw_bits = static_cast<uint16_t>((bits + 0x7FFFu + lsb) >> 16);
    }

    /// Widen to float (exact).
    operator float() const {
        const uint32_t bits = static_cast<uint32_t>(raw_bits) << 16;
        float f;
        std::memcpy(&f, &bits, sizeof f);
        return f;
    }

    bfloat16_t& operator=(float f) {
        *this = bfloat16_t(f);
        return *this;
    }
};

static_assert(sizeof(bfloat16_t) == 2, "bfloat16_t must be 2 bytes");

/// Per-call algorithm override for gemm_fp32.
///
/// On this implementation kAuto runs the gfx950 shape dispatcher and kNaive
/// runs the one-thread-per-output device kernel that reproduces the scalar
/// reference loop bit for bit (no fused multiply-add).  Every other value is
/// an ISA-specific request of the reference (NEON/SVE/SME/FP8 kernels) and is
/// served by the dispatcher exactly like kAuto.
enum class GemmAlgo {
    kAuto,
    kNaive,
    kNeonFp32,
    kBf16Bfmmla,
    kInt8Smmla,
    kInt8Sdot,
    kSveFp32,
    kSveBf16,
    kSveInt8,
    kSmeFp32,
    kFp8E4m3Fdot,
    kFp8E5m2Fdot,
    kSveFp8E4m3,
    kSveFp8E5m2,
};

}  // namespace dnnopt
