// One 16 x 16 output tile of y = x W^T (+ bias) on the fp32 / bf16 matrix
// cores, in the form of the one-wave-per-tile linear (linear_small_kernel in
// linear.hip): lane l = 16 g + i holds x row i and W row i, k = 32 s + 8 g ..
// + 7 of every 32-wide k step s, and receives y[row i][cols 4g .. 4g + 3].
// The helpers are shared with the fused RMSNorm -> Mamba-3 block kernel so
// that its in_proj and out_proj tiles are computed by the same instruction
// sequence, and therefore equal the separate operators' results bit for bit.
#pragma once

#include "mlk_common.h"

namespace mlk {

typedef float tile_f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 tile_bf16x8 __attribute__((ext_vector_type(8)));

// The 8 floats src[k0 .. k0 + 7] (k0 = 32 s + 8 g) of KS steps into v; a
// step whose k0 lies past K (live false) reads offset 0 instead and its values
// are zeroed where consumed. src must be 16-byte aligned with K % 8 == 0.
template <int KS>
__device__ __forceinline__ void tile_load8(const float* src, int K, int group, float (&v)[KS][8], bool (&live)[KS]) {
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        const int k = 32 * s + 8 * group;
        live[s] = k < K;
        const float* p = src + (live[s] ? k : 0);
        const float4 lo = *reinterpret_cast<const float4*>(p);
        const float4 hi = *reinterpret_cast<const float4*>(p + 4);
        v[s][0] = lo.x; v[s][1] = lo.y; v[s][2] = lo.z; v[s][3] = lo.w;
        v[s][4] = hi.x; v[s][5] = hi.y; v[s][6] = hi.z; v[s][7] = hi.w;
    }
}

// The grouped RMSNorm (groups of GS floats, GS in 8, 16, 32, 64) of the
// loaded x fragments, with the arithmetic of rms_norm_vec_kernel: per 4-float
// chunk the fp64 partial (a^2 + b^2) + (c^2 + d^2), the group's chunks
// combined by the same butterfly (chunk c of the group is lane (c / 2) % 4's
// half c % 2 of its segment, so the levels are: the two steps of a 64-group
// in registers, lanes 32 apart, lanes 16 apart, the two halves in
// registers), scale = 1 / sqrt(sum / GS + eps), x * scale * w rounded once.
// nw holds the norm weight fragments loaded like x.
template <int KS, int GS>
__device__ __forceinline__ void tile_rms_norm(float (&xv)[KS][8], const float (&nw)[KS][8], double eps) {
    static_assert(GS == 8 || GS == 16 || GS == 32 || (GS == 64 && KS % 2 == 0), "RMSNorm group size");
    double part[KS][2];
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const double a = xv[s][4 * hf], b = xv[s][4 * hf + 1], c = xv[s][4 * hf + 2], d = xv[s][4 * hf + 3];
            part[s][hf] = (a * a + b * b) + (c * c + d * d);
        }
    if constexpr (GS == 64) {
#pragma unroll
        for (int s = 0; s < KS; s += 2)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                const double q = part[s][hf] + part[s + 1][hf];
                part[s][hf] = q;
                part[s + 1][hf] = q;
            }
    }
    if constexpr (GS >= 32) {
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) part[s][hf] += shfl_xor_d(part[s][hf], 32);
    }
    if constexpr (GS >= 16) {
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) part[s][hf] += shfl_xor_d(part[s][hf], 16);
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        const double scale = 1.0 / sqrt((part[s][0] + part[s][1]) / static_cast<double>(GS) + eps);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            xv[s][j] = static_cast<float>((static_cast<double>(xv[s][j]) * scale) * static_cast<double>(nw[s][j]));
        }
    }
}

// The tile's products with fp32 weights: W as the A operand (so the result is
// transposed into the lane layout above), the even and odd k of each lane in
// two accumulation chains, summed at the end. ALL_LIVE (K = 32 KS, every step
// live) takes the operands as loaded: the same products, without the select
// in front of every MFMA, whose VALU -> MFMA operand hazard otherwise halves
// the issue rate.
template <int KS, bool ALL_LIVE = false>
__device__ __forceinline__ tile_f32x4 tile_mfma_f32(const float (&wv)[KS][8], const float (&xv)[KS][8],
                                                   const bool (&live)[KS]) {
    tile_f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f};
    tile_f32x4 acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        const bool on = ALL_LIVE || live[s];
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(on ? wv[s][j] : 0.0f, on ? xv[s][j] : 0.0f, acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(on ? wv[s][j + 1] : 0.0f, on ? xv[s][j + 1] : 0.0f, acc1, 0,
                                                        0, 0);
        }
    }
    return acc0 + acc1;
}

// Two tiles against the same x fragments, their four chains interleaved (each
// tile's products and sums exactly as tile_mfma_f32 forms them).
template <int KS, bool ALL_LIVE = false>
__device__ __forceinline__ void tile_mfma_f32_pair(const float (&wa)[KS][8], const float (&wb)[KS][8],
                                                   const float (&xv)[KS][8], const bool (&live)[KS], tile_f32x4& ya,
                                                   tile_f32x4& yb) {
    tile_f32x4 a0 = {0.0f, 0.0f, 0.0f, 0.0f}, a1 = a0, b0 = a0, b1 = a0;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        const bool on = ALL_LIVE || live[s];
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            const float x0 = on ? xv[s][j] : 0.0f, x1 = on ? xv[s][j + 1] : 0.0f;
            a0 = __builtin_amdgcn_mfma_f32_16x16x4f32(on ? wa[s][j] : 0.0f, x0, a0, 0, 0, 0);
            b0 = __builtin_amdgcn_mfma_f32_16x16x4f32(on ? wb[s][j] : 0.0f, x0, b0, 0, 0, 0);
            a1 = __builtin_amdgcn_mfma_f32_16x16x4f32(on ? wa[s][j + 1] : 0.0f, x1, a1, 0, 0, 0);
            b1 = __builtin_amdgcn_mfma_f32_16x16x4f32(on ? wb[s][j + 1] : 0.0f, x1, b1, 0, 0, 0);
        }
    }
    ya = a0 + a1;
    yb = b0 + b1;
}

}  // namespace mlk
