// Shared helpers of the MI355X (gfx950) RDT4quant kernels: the status /
// last-error convention of the C ABI and small device utilities.
//
// Status convention (mirrors montlok_status + a thread-local last error,
// include/montlok/montlok.h:16-17,43-52 of the reference): every entry point
// returns an mlk_status; on failure mlk_last_error() names the argument or
// the HIP call that failed, with the same wording as the reference's
// TORCH_CHECK messages where one exists.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/mlk_hip.h"

namespace mlk {

void set_error(const std::string& message);
void clear_error();

// Validation helper: `MLK_CHECK(cond, "message")` returns MLK_ERR_INVALID_ARGUMENT.
#define MLK_CHECK(cond, msg)                                   \
    do {                                                       \
        if (!(cond)) {                                         \
            ::mlk::set_error(msg);                             \
            return MLK_ERR_INVALID_ARGUMENT;                   \
        }                                                      \
    } while (0)

// Kernel launch epilogue: turns a launch error into MLK_ERR_RUNTIME.
mlk_status launch_status(const char* what);

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// Device utilities
// ---------------------------------------------------------------------------

constexpr int kWave = 64;

__device__ __forceinline__ double shfl_xor_d(double v, int mask) { return __shfl_xor(v, mask, kWave); }

// A double moved between lanes by one DPP control (GFX9 encodings: quad_perm
// 0x00-0xFF, row_mirror 0x140, row_half_mirror 0x141), both halves alike.
template <int CTRL>
__device__ __forceinline__ double mov_dpp_d(double v) {
    const int lo = __builtin_amdgcn_mov_dpp(__double2loint(v), CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_mov_dpp(__double2hiint(v), CTRL, 0xF, 0xF, false);
    return __hiloint2double(hi, lo);
}

// The value of lane l ^ MASK, MASK in {1, 2, 4, 8} (a partner inside the
// lane's row of 16), by DPP moves instead of the LDS crossbar: quad_perm
// [1,0,3,2] for 1, [2,3,0,1] for 2; row_half_mirror (l ^ 7) then quad_perm
// [3,2,1,0] (l ^ 3) for 4; row_mirror (l ^ 15) then row_half_mirror for 8.
// The same partner as shfl_xor_d(v, MASK), so sums built from it agree bit
// for bit.
template <int MASK>
__device__ __forceinline__ double xor_row_d(double v) {
    static_assert(MASK == 1 || MASK == 2 || MASK == 4 || MASK == 8, "partner must lie in the 16-lane row");
    if constexpr (MASK == 1) return mov_dpp_d<0xB1>(v);
    if constexpr (MASK == 2) return mov_dpp_d<0x4E>(v);
    if constexpr (MASK == 4) return mov_dpp_d<0x1B>(mov_dpp_d<0x141>(v));
    return mov_dpp_d<0x141>(mov_dpp_d<0x140>(v));
}
__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, kWave); }
__device__ __forceinline__ double shfl_d(double v, int src) { return __shfl(v, src, kWave); }

// ---------------------------------------------------------------------------
// Double-precision exp / tanh / sigmoid with short dependency chains
// ---------------------------------------------------------------------------
//
// exp(x): Cody-Waite reduction x = k ln2 + r with the two-part ln2 of fdlibm
// (hi has 32 significant bits, so k * hi is exact for |k| < 2^21), |r| <=
// ln2 / 2, then the degree-13 Taylor polynomial of e^r (truncation below
// 4e-18 relative on that interval) evaluated with Estrin's scheme (about six
// dependent operations instead of thirteen for Horner), scaled by 2^k with
// ldexp (which also produces the overflow to +inf above ~709.78 and the
// underflow to 0). Agrees with a correctly rounded exp to a couple of double
// ulp; after rounding to float32 the results agree with it except in rare
// ties.
// exp_d_core takes x in [-746, 710] (NaN passes through as NaN); exp_d clamps first.
__device__ __forceinline__ double exp_d_core(double x) {
    const double kf = __builtin_rint(x * 1.4426950408889634074);
    const double r = fma(-kf, 1.90821492927058770002e-10, fma(-kf, 6.93147180369123816490e-01, x));
    const double r2 = r * r;
    const double r4 = r2 * r2;
    const double r8 = r4 * r4;
    // 1/i! for i = 0..13
    const double p01 = fma(r, 1.0, 1.0);
    const double p23 = fma(r, 1.0 / 6.0, 0.5);
    const double p45 = fma(r, 1.0 / 120.0, 1.0 / 24.0);
    const double p67 = fma(r, 1.0 / 5040.0, 1.0 / 720.0);
    const double p89 = fma(r, 1.0 / 362880.0, 1.0 / 40320.0);
    const double pab = fma(r, 1.0 / 39916800.0, 1.0 / 3628800.0);
    const double pcd = fma(r, 1.0 / 6227020800.0, 1.0 / 479001600.0);
    const double q0 = fma(p23, r2, p01);
    const double q1 = fma(p67, r2, p45);
    const double q2 = fma(pab, r2, p89);
    const double s0 = fma(q1, r4, q0);
    const double s1 = fma(pcd, r4, q2);
    const double poly = fma(s1, r8, s0);
    return __builtin_ldexp(poly, static_cast<int>(kf));
}
__device__ __forceinline__ double exp_d(double x) {
    // Outside [-746, 710] the result is 0 or +inf; the comparisons keep NaN.
    x = x < -746.0 ? -746.0 : (x > 710.0 ? 710.0 : x);
    return exp_d_core(x);
}

// 1 / x for positive normal x (also 1 / inf = 0): the hardware reciprocal
// (relative error ~5e-8) refined by two Newton steps r += r (1 - x r). Over
// 2^18 inputs in [0.5, 4) the result equalled the IEEE quotient every time;
// it is within a double ulp by construction. recip_finite is the same steps
// without the infinity test, for callers that know x is finite.
__device__ __forceinline__ double recip_finite(double x) {
    double r = __builtin_amdgcn_rcp(x);
    double e = fma(-x, r, 1.0);
    r = fma(r, e, r);
    e = fma(-x, r, 1.0);
    return fma(r, e, r);
}
__device__ __forceinline__ double recip_pos(double x) {
    return __builtin_isinf(x) ? 0.0 : recip_finite(x);
}

// tanh(x) = sign(x) (1 - t) / (1 + t), t = exp(-2 |x|) in (0, 1]: absolute
// error a few 1e-16 (the consumers add it to an O(1) bias).
__device__ __forceinline__ double tanh_d(double x) {
    // (the exponent is never positive: only exp_d's lower clamp can bind, and a NaN passes through it)
    const double m = -2.0 * __builtin_fabs(x);
    const double t = exp_d_core(m < -746.0 ? -746.0 : m);
    const double y = (1.0 - t) * recip_pos(1.0 + t);
    return __builtin_copysign(y, x);
}

// 1 / (1 + exp(-x)).
__device__ __forceinline__ double sigmoid_fast(double x) { return recip_pos(1.0 + exp_d(-x)); }

// The output gate silu(z) = z / (1 + exp(-z)) in double, formed as z times the reciprocal of 1 + exp(-z)
// (recip_pos: within a double ulp of the quotient, 1 / inf = 0): the IEEE division's scaling and fix-up
// steps cost the stack's scan 3.5% of its time, and the product differs from the quotient by at most an
// ulp of a double, far below the float32 rounding the gated output takes next.
// exp(-z)'s argument is clamped to [-746, 710] by min/max, two instructions where exp_d's NaN-keeping
// selects take six: a NaN z then takes exp(710) = inf instead of exp(NaN), and the gate is z * 0 = NaN
// either way, so the result equals the select form's for every z.
__device__ __forceinline__ double silu_d(double z) {
    const double x = __builtin_fmax(__builtin_fmin(-z, 710.0), -746.0);
    return z * recip_pos(1.0 + exp_d_core(x));
}

// sin and cos of x in double for |x| below a few multiples of pi (the Mamba
// rotary phases are wrapped to [0, 2pi) before this call). Cody-Waite
// reduction by pi/2 with fdlibm's two-part constant (pio2_1 carries 33
// significant bits, so k * pio2_1 is exact for the small quadrant counts k
// here) to r in [-pi/4, pi/4], then the Taylor series of sin to r^15 and of
// cos to r^16 (truncation below 1e-16 relative at |r| = pi/4), evaluated in
// r^2 with Estrin's scheme, and the quadrant swap/negation. Results agree
// with a correctly rounded sin/cos to a couple of double ulp.
__device__ __forceinline__ void sincos_d(double x, double* sine, double* cosine) {
    const double kf = __builtin_rint(x * 0.63661977236758134308);
    const double r = fma(-kf, 6.07710050650619224932e-11, fma(-kf, 1.57079632673412561417e+00, x));
    const double z = r * r;
    const double z2 = z * z;
    const double z4 = z2 * z2;
    // sin(r) = r * P(z), P(z) = sum_i (-1)^i z^i / (2i+1)!, i = 0..7
    const double s01 = fma(z, -1.0 / 6.0, 1.0);
    const double s23 = fma(z, -1.0 / 5040.0, 1.0 / 120.0);
    const double s45 = fma(z, -1.0 / 39916800.0, 1.0 / 362880.0);
    const double s67 = fma(z, -1.0 / 1307674368000.0, 1.0 / 6227020800.0);
    const double sp = fma(fma(s67, z2, s45), z4, fma(s23, z2, s01));
    // cos(r) = Q(z), Q(z) = sum_i (-1)^i z^i / (2i)!, i = 0..8
    const double c01 = fma(z, -0.5, 1.0);
    const double c23 = fma(z, -1.0 / 720.0, 1.0 / 24.0);
    const double c45 = fma(z, -1.0 / 3628800.0, 1.0 / 40320.0);
    const double c67 = fma(z, -1.0 / 87178291200.0, 1.0 / 479001600.0);
    const double c8 = 1.0 / 20922789888000.0;
    const double cq = fma(fma(fma(c8, z2, c67), z2, c45), z4, fma(c23, z2, c01));
    const double sr = r * sp;
    const int quadrant = static_cast<int>(kf) & 3;
    double so = (quadrant & 1) ? cq : sr;
    double co = (quadrant & 1) ? -sr : cq;
    if (quadrant & 2) {
        so = -so;
        co = -co;
    }
    *sine = so;
    *cosine = co;
}

// Sum over aligned groups of `width` lanes (width a power of two <= 64);
// every lane of a group receives the group total.
template <int width>
__device__ __forceinline__ double group_sum_d(double v) {
#pragma unroll
    for (int mask = width / 2; mask > 0; mask >>= 1) {
        v += shfl_xor_d(v, mask);
    }
    return v;
}

}  // namespace mlk
