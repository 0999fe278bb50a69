// Fixed-point requantization of the INT8 configuration with int8 tensors
// between nodes, shared by the device kernels and a host test build.
//
// Definition (one rounding): for an int32 accumulator sum(w (x - z_x)) acc,
// per-channel constants c (bias_q folded in), multipliers m1, m2 and shift
// S in [1, 62], and the residual's int8 value minus its zero point rd,
//   t = (acc + c) m1 + rd m2            (exact, int64)
//   q = round_half_away(t / 2^S) + z_y, Relu as max(q, z_y), saturated to int8.
// round_half_away(t / 2^S) = (t + 2^(S-1) - [t < 0]) >> S (arithmetic shift).
//
// q8_requant computes it with 64-bit shifts; q8_requant_hi computes the same
// for S in [33, 55] from the high word of t alone: with k = S - 32 and half =
// 2^(k-1), the multiply-add folds half into the high word (t + half 2^32 has
// high word hi(t) + half, the low word untouched), and the low word only
// decides a borrow for negative t whose low word is 0 (t + 2^(S-1) - 1
// borrows from the high word exactly then), so the rounding and shift are
// 32-bit operations.
// |acc + c| < 2^31 is guaranteed by the callers (K <= 32768 bytes, |bias_q|
// <= 2^30), so acc + c is a 32-bit sum and each product one signed 32 x 32
// multiply-add.
#pragma once

#include <cstdint>

#if defined(__HIPCC__)
#define Q8_HD __host__ __device__ __forceinline__
#else
#define Q8_HD inline
#endif

namespace spk::kern {

Q8_HD int q8_clamp(int v, int lo) {
    const int u = v < 127 ? v : 127;
    return u > lo ? u : lo;
}

// lo: the clamp's lower end, z_y with Relu, -128 without
Q8_HD int q8_requant(int acc, int c, int m1, int m2, int sh, int rd, int zy, int lo) {
    const int64_t t = static_cast<int64_t>(acc + c) * m1 + static_cast<int64_t>(rd) * m2;
    const int64_t half = int64_t(1) << (sh - 1);
    return q8_clamp(static_cast<int>((t + half - (t < 0 ? 1 : 0)) >> sh) + zy, lo);
}

// S in [33, 55]: k = S - 32 in [1, 23], halfz = 2^(k-1) + z_y 2^k (the
// output zero point folded in: adding a multiple of 2^k before the shift adds
// z_y after it); `clamp(v, lo)` saturates to [lo, 127].
template <class Clamp>
Q8_HD int q8_requant_hi(int acc, int c, int m1, int m2, int halfz, int k, int rd, int lo, Clamp clamp) {
    const int64_t t = static_cast<int64_t>(acc + c) * m1 + (static_cast<int64_t>(halfz) << 32) +
                      static_cast<int64_t>(rd) * m2;
    const int hi = static_cast<int>(t >> 32);  // hi(true t) + halfz
    const unsigned lw = static_cast<unsigned>(t);
    const int borrow = (hi < halfz && lw == 0u) ? 1 : 0;  // true t < 0 with a zero low word
    return clamp((hi - borrow) >> k, lo);
}

}  // namespace spk::kern
