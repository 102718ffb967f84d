// Row-wise layers of the RDT4quant path on gfx950: RMSNorm / GroupedRMSNorm,
// add + RMSNorm, LayerNorm and the SwiGLU gate.
//
// Semantics (reference rdt4quant_cpu/montlok_layers.h): every intermediate is
// evaluated in double and the output rounded to float32 once; eps is the
// Python float cast through float32 (montlok.cpp:932, :1000, :1076).
//   RMSNorm   out = (x * (1 / sqrt(sum(x^2) / gs + eps))) * w   per group of gs
//   LayerNorm out = ((x - mean) * (1 / sqrt(var + eps))) * w + b (biased var)
//   SwiGLU    out = (g / (1 + exp(-g))) * u
// The squares of fp32 inputs are exact in double, so the RMSNorm result does
// not depend on the summation order except through the final rounding of the
// double sum.
//
// Mapping: a group of `gs` floats is held by LPG lanes (a power of two up to
// 64), each lane owning CPL float4 chunks; the group sum is a butterfly over
// the LPG lanes. One 256-thread block covers 256 / LPG groups. Rows whose
// group size, stride or alignment do not allow float4 access fall back to a
// one-wave-per-group kernel with scalar loads. All kernels are HBM-bound:
// algorithmic traffic is one read of x (and w, from cache) and one write.
#include "mlk_common.h"

namespace mlk {
namespace {

constexpr int kBlock = 256;
#ifndef MLK_NORM_RPW
#define MLK_NORM_RPW 4
#endif
constexpr int kNormRpw = MLK_NORM_RPW;  // rows per lane group in large launches

// RPW groups per lane group, one after the other in the arithmetic but with
// all their loads issued first: a wave then has RPW times the bytes in flight
// and a block RPW times the work (262144 rows of 256: one row per wave left the
// kernel at 46% of HBM, its waves each waiting on one 16-byte load per lane).
// Group r of block b's lane group k is (b RPW + r) (256 / LPG) + k, so each
// load instruction still reads the block's groups side by side. Per group the
// arithmetic is unchanged.
template <int LPG, int CPL, bool ADD, int RPW = 1>
__global__ __launch_bounds__(kBlock) void rms_norm_vec_kernel(const float* __restrict__ x,
                                                              const float* __restrict__ right,
                                                              const float* __restrict__ w, int64_t total_groups,
                                                              int64_t groups, int64_t gs, int64_t dim,
                                                              int64_t row_stride, double eps,
                                                              float* __restrict__ residual, float* __restrict__ out) {
    const int li = threadIdx.x % LPG;
    int64_t gid[RPW], row[RPW], g[RPW];
    bool active[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        gid[r] = (static_cast<int64_t>(blockIdx.x) * RPW + r) * (kBlock / LPG) + threadIdx.x / LPG;
        active[r] = gid[r] < total_groups;
        // One group per row (the plain RMSNorm) skips the 64-bit division, whose slow path sat in front of
        // every load (262144 x 256: 116 -> 106 us); group counts below 2^31 divide in 32 bits.
        if (groups == 1) {
            row[r] = active[r] ? gid[r] : 0;
            g[r] = 0;
        } else if (total_groups < (int64_t{1} << 31)) {
            const unsigned gu = static_cast<unsigned>(active[r] ? gid[r] : 0), gn = static_cast<unsigned>(groups);
            row[r] = gu / gn;
            g[r] = gu % gn;
        } else {
            row[r] = active[r] ? gid[r] / groups : 0;
            g[r] = active[r] ? gid[r] % groups : 0;
        }
    }
    // Every load is issued before the first use, without a branch around it:
    // lanes past the last group read group 0 (in bounds); all LPG lanes of a
    // group share `active`, so those sums never meet a live group's.
    float4 v[RPW][CPL], wv[RPW][CPL];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const float* xg = x + row[r] * row_stride + g[r] * gs;
#pragma unroll
        for (int c = 0; c < CPL; ++c) v[r][c] = *reinterpret_cast<const float4*>(xg + static_cast<int64_t>(c * LPG + li) * 4);
    }
    if constexpr (ADD) {
        float4 rv[RPW][CPL];
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int c = 0; c < CPL; ++c)
                rv[r][c] = *reinterpret_cast<const float4*>(right + row[r] * row_stride + g[r] * gs +
                                                            static_cast<int64_t>(c * LPG + li) * 4);
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                v[r][c].x += rv[r][c].x;
                v[r][c].y += rv[r][c].y;
                v[r][c].z += rv[r][c].z;
                v[r][c].w += rv[r][c].w;
                if (active[r]) {
                    *reinterpret_cast<float4*>(residual + row[r] * dim + g[r] * gs + static_cast<int64_t>(c * LPG + li) * 4) =
                        v[r][c];
                }
            }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int c = 0; c < CPL; ++c)
            wv[r][c] = *reinterpret_cast<const float4*>(w + g[r] * gs + static_cast<int64_t>(c * LPG + li) * 4);
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        double sumsq = 0.0;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const double a = v[r][c].x, b = v[r][c].y, cc = v[r][c].z, d = v[r][c].w;
            sumsq += (a * a + b * b) + (cc * cc + d * d);
        }
        sumsq = group_sum_d<LPG>(sumsq);
        if (!active[r]) continue;
        const double scale = 1.0 / sqrt(sumsq / static_cast<double>(gs) + eps);
        float* og = out + row[r] * dim + g[r] * gs;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int64_t off = static_cast<int64_t>(c * LPG + li) * 4;
            const float4 wv_c = wv[r][c];
            float4 o;
            o.x = static_cast<float>((static_cast<double>(v[r][c].x) * scale) * static_cast<double>(wv_c.x));
            o.y = static_cast<float>((static_cast<double>(v[r][c].y) * scale) * static_cast<double>(wv_c.y));
            o.z = static_cast<float>((static_cast<double>(v[r][c].z) * scale) * static_cast<double>(wv_c.z));
            o.w = static_cast<float>((static_cast<double>(v[r][c].w) * scale) * static_cast<double>(wv_c.w));
            *reinterpret_cast<float4*>(og + off) = o;
        }
    }
}

// One wave per group, scalar loads: any group size, stride and alignment.
template <bool ADD>
__global__ __launch_bounds__(kBlock) void rms_norm_scalar_kernel(const float* __restrict__ x,
                                                                 const float* __restrict__ right,
                                                                 const float* __restrict__ w, int64_t total_groups,
                                                                 int64_t groups, int64_t gs, int64_t dim,
                                                                 int64_t row_stride, double eps,
                                                                 float* __restrict__ residual,
                                                                 float* __restrict__ out) {
    const int64_t gid = static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (gid >= total_groups) return;  // whole waves exit together
    const int64_t row = gid / groups;
    const int64_t g = gid % groups;
    const float* xg = x + row * row_stride + g * gs;
    double sumsq = 0.0;
    for (int64_t k = lane; k < gs; k += kWave) {
        float v = xg[k];
        if constexpr (ADD) {
            v += right[row * row_stride + g * gs + k];
            residual[row * dim + g * gs + k] = v;
        }
        sumsq += static_cast<double>(v) * static_cast<double>(v);
    }
    sumsq = group_sum_d<kWave>(sumsq);
    const double scale = 1.0 / sqrt(sumsq / static_cast<double>(gs) + eps);
    for (int64_t k = lane; k < gs; k += kWave) {
        float v = xg[k];
        if constexpr (ADD) v += right[row * row_stride + g * gs + k];
        out[row * dim + g * gs + k] =
            static_cast<float>((static_cast<double>(v) * scale) * static_cast<double>(w[g * gs + k]));
    }
}

template <bool ADD>
mlk_status launch_rms(const float* x, const float* right, const float* w, int64_t rows, int64_t dim,
                      int64_t row_stride, double eps, int64_t groups, float* residual, float* out,
                      hipStream_t stream) {
    const int64_t gs = dim / groups;
    const int64_t total = rows * groups;
    if (total == 0) return MLK_OK;
    const double eps_f = static_cast<double>(static_cast<float>(eps));
    const bool aligned = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && (reinterpret_cast<uintptr_t>(w) % 16 == 0) &&
                         (reinterpret_cast<uintptr_t>(out) % 16 == 0) && row_stride % 4 == 0 && gs % 4 == 0 &&
                         (!ADD || (reinterpret_cast<uintptr_t>(right) % 16 == 0 &&
                                   reinterpret_cast<uintptr_t>(residual) % 16 == 0));
    const int64_t chunks = gs / 4;
    // Four groups per lane group where one each would take 4096 blocks or more.
#define MLK_RMS_VEC(LPG, CPL)                                                                                \
    do {                                                                                                     \
        const int64_t blocks = ceil_div(total, kBlock / (LPG));                                              \
        if (blocks >= 4096) {                                                                                \
            hipLaunchKernelGGL((rms_norm_vec_kernel<LPG, CPL, ADD, kNormRpw>), dim3(ceil_div(blocks, kNormRpw)), dim3(kBlock), \
                               0, stream, x, right, w, total, groups, gs, dim, row_stride, eps_f, residual, out); \
        } else {                                                                                             \
            hipLaunchKernelGGL((rms_norm_vec_kernel<LPG, CPL, ADD>), dim3(blocks), dim3(kBlock), 0, stream, x, \
                               right, w, total, groups, gs, dim, row_stride, eps_f, residual, out);          \
        }                                                                                                    \
        return launch_status("rms_norm");                                                                    \
    } while (0)
    if (aligned) {
        switch (chunks) {
            case 1: MLK_RMS_VEC(1, 1);
            case 2: MLK_RMS_VEC(2, 1);
            case 4: MLK_RMS_VEC(4, 1);
            case 8: MLK_RMS_VEC(8, 1);
            case 16: MLK_RMS_VEC(16, 1);
            case 32: MLK_RMS_VEC(32, 1);
            case 64: MLK_RMS_VEC(64, 1);
            case 128: MLK_RMS_VEC(64, 2);
            case 256: MLK_RMS_VEC(64, 4);
            default: break;
        }
    }
#undef MLK_RMS_VEC
    const int64_t blocks = ceil_div(total, kBlock / kWave);
    hipLaunchKernelGGL((rms_norm_scalar_kernel<ADD>), dim3(blocks), dim3(kBlock), 0, stream, x, right, w, total,
                       groups, gs, dim, row_stride, eps_f, residual, out);
    return launch_status("rms_norm");
}

// LayerNorm: one wave per row, the row held in registers as float4 chunks
// when possible (two passes over registers: mean, then centred squares).
// BF16OUT: the float results rounded once more to bf16 (round to nearest
// even), written as bf16 rows of dim.
template <int CPL, bool BF16OUT = false, int RPW = 1>
__global__ __launch_bounds__(kBlock) void layer_norm_vec_kernel(const float* __restrict__ x,
                                                                const float* __restrict__ w,
                                                                const float* __restrict__ bias, int64_t rows,
                                                                int64_t dim, int64_t row_stride, double eps,
                                                                void* __restrict__ out) {
    // LPG lanes per row: dim = 4 * CPL * LPG with LPG = 64 / rows-per-wave. RPW rows per lane group, all
    // their loads issued first (as rms_norm_vec_kernel): row r of block b's lane group k is
    // (b RPW + r) (256 / LPG) + k.
    const int lpg = static_cast<int>(dim / (4 * CPL));
    const int li = threadIdx.x % lpg;
    int64_t row[RPW];
    bool active[RPW];
    // Loads first, unconditional (rows past the end read row 0; a row's lanes
    // share `active`), weights and bias with them.
    float4 v[RPW][CPL], wv[CPL], bv[CPL];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        row[r] = (static_cast<int64_t>(blockIdx.x) * RPW + r) * (kBlock / lpg) + threadIdx.x / lpg;
        active[r] = row[r] < rows;
        const float* xr = x + (active[r] ? row[r] : 0) * row_stride;
#pragma unroll
        for (int c = 0; c < CPL; ++c) v[r][c] = *reinterpret_cast<const float4*>(xr + (c * lpg + li) * 4);
    }
    const float* bsrc = bias != nullptr ? bias : w;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        wv[c] = *reinterpret_cast<const float4*>(w + (c * lpg + li) * 4);
        bv[c] = *reinterpret_cast<const float4*>(bsrc + (c * lpg + li) * 4);
        if (bias == nullptr) bv[c] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const double inv_dim = 1.0 / static_cast<double>(dim);
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        double sum = 0.0;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            sum += (static_cast<double>(v[r][c].x) + static_cast<double>(v[r][c].y)) +
                   (static_cast<double>(v[r][c].z) + static_cast<double>(v[r][c].w));
        }
        for (int mask = lpg / 2; mask > 0; mask >>= 1) sum += shfl_xor_d(sum, mask);
        const double mean = sum * inv_dim;
        double sumsq = 0.0;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const double a = static_cast<double>(v[r][c].x) - mean, b = static_cast<double>(v[r][c].y) - mean;
            const double cc = static_cast<double>(v[r][c].z) - mean, d = static_cast<double>(v[r][c].w) - mean;
            sumsq += (a * a + b * b) + (cc * cc + d * d);
        }
        for (int mask = lpg / 2; mask > 0; mask >>= 1) sumsq += shfl_xor_d(sumsq, mask);
        if (!active[r]) continue;
        const double rstd = 1.0 / sqrt(fma(sumsq, inv_dim, eps));
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int off = (c * lpg + li) * 4;
            float4 o;
            o.x = static_cast<float>(((static_cast<double>(v[r][c].x) - mean) * rstd) * wv[c].x + static_cast<double>(bv[c].x));
            o.y = static_cast<float>(((static_cast<double>(v[r][c].y) - mean) * rstd) * wv[c].y + static_cast<double>(bv[c].y));
            o.z = static_cast<float>(((static_cast<double>(v[r][c].z) - mean) * rstd) * wv[c].z + static_cast<double>(bv[c].z));
            o.w = static_cast<float>(((static_cast<double>(v[r][c].w) - mean) * rstd) * wv[c].w + static_cast<double>(bv[c].w));
            if constexpr (BF16OUT) {
                auto hb = [](float f) { return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(f))); };
                *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + row[r] * dim + off) =
                    make_uint2(hb(o.x) | (hb(o.y) << 16), hb(o.z) | (hb(o.w) << 16));
            } else {
                *reinterpret_cast<float4*>(static_cast<float*>(out) + row[r] * dim + off) = o;
            }
        }
    }
}

__global__ __launch_bounds__(kBlock) void layer_norm_scalar_kernel(const float* __restrict__ x,
                                                                   const float* __restrict__ w,
                                                                   const float* __restrict__ bias, int64_t rows,
                                                                   int64_t dim, int64_t row_stride, double eps,
                                                                   float* __restrict__ out) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (row >= rows) return;
    const float* xr = x + row * row_stride;
    double sum = 0.0;
    for (int64_t k = lane; k < dim; k += kWave) sum += static_cast<double>(xr[k]);
    sum = group_sum_d<kWave>(sum);
    const double inv_dim = 1.0 / static_cast<double>(dim);
    const double mean = sum * inv_dim;
    double sumsq = 0.0;
    for (int64_t k = lane; k < dim; k += kWave) {
        const double a = static_cast<double>(xr[k]) - mean;
        sumsq += a * a;
    }
    sumsq = group_sum_d<kWave>(sumsq);
    const double rstd = 1.0 / sqrt(fma(sumsq, inv_dim, eps));
    for (int64_t k = lane; k < dim; k += kWave) {
        double y = ((static_cast<double>(xr[k]) - mean) * rstd) * static_cast<double>(w[k]);
        if (bias != nullptr) y += static_cast<double>(bias[k]);
        out[row * dim + k] = static_cast<float>(y);
    }
}

template <typename I>
__global__ __launch_bounds__(kBlock) void swiglu_kernel(const float* __restrict__ x, int64_t rows, int64_t hidden,
                                                        int64_t row_stride, float* __restrict__ out) {
    const I i = static_cast<I>(blockIdx.x) * kBlock + threadIdx.x;
    if (static_cast<int64_t>(i) >= rows * hidden) return;
    const I row_i = i / static_cast<I>(hidden);
    const int64_t row = row_i;
    const int64_t k = i - row_i * static_cast<I>(hidden);
    const double z = static_cast<double>(x[row * row_stride + k]);
    const double u = static_cast<double>(x[row * row_stride + hidden + k]);
    out[i] = static_cast<float>((z / (1.0 + exp(-z))) * u);
}

}  // namespace
}  // namespace mlk

using namespace mlk;

extern "C" {

mlk_status mlk_rms_norm(const float* x, int64_t rows, int64_t dim, int64_t row_stride, const float* weight,
                        double eps, int64_t groups, float* out, mlk_stream_t stream) {
    MLK_CHECK(rows >= 0 && dim >= 1, "x must have at least one dimension");
    MLK_CHECK(groups > 0 && dim % groups == 0, "groups must divide the normalised dimension");
    MLK_CHECK(rows == 0 || (x != nullptr && weight != nullptr && out != nullptr), "null tensor pointer");
    MLK_CHECK(row_stride >= dim || rows <= 1, "x rows overlap");
    return launch_rms<false>(x, nullptr, weight, rows, dim, row_stride, eps, groups, nullptr, out, stream);
}

mlk_status mlk_add_rms_norm(const float* left, const float* right, int64_t rows, int64_t dim, const float* weight,
                            double eps, int64_t groups, float* residual, float* normalized, mlk_stream_t stream) {
    MLK_CHECK(rows >= 0 && dim >= 1, "residual operands must have the same shape");
    MLK_CHECK(groups > 0 && dim % groups == 0, "groups must divide the normalized dimension");
    MLK_CHECK(rows == 0 || (left && right && weight && residual && normalized), "null tensor pointer");
    return launch_rms<true>(left, right, weight, rows, dim, dim, eps, groups, residual, normalized, stream);
}

mlk_status mlk_layer_norm(const float* x, int64_t rows, int64_t dim, int64_t row_stride, const float* weight,
                          const float* bias, double eps, float* out, mlk_stream_t stream) {
    MLK_CHECK(rows >= 0 && dim >= 1, "x must have at least one dimension");
    MLK_CHECK(rows == 0 || (x != nullptr && weight != nullptr && out != nullptr), "null tensor pointer");
    if (rows == 0) return MLK_OK;
    const double eps_f = static_cast<double>(static_cast<float>(eps));
    const bool aligned = reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(weight) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(out) % 16 == 0 &&
                         (bias == nullptr || reinterpret_cast<uintptr_t>(bias) % 16 == 0) && row_stride % 4 == 0;
    // dim = 4 * CPL * lpg with lpg a power of two <= 64.
    int cpl = 0;
    if (aligned && dim % 4 == 0) {
        const int64_t chunks = dim / 4;
        if (chunks <= 64 && (chunks & (chunks - 1)) == 0) cpl = 1;
        else if (chunks == 128) cpl = 2;
        else if (chunks == 256) cpl = 4;
    }
    if (cpl > 0) {
        const int lpg = static_cast<int>(dim / (4 * cpl));
        const int64_t blocks = ceil_div(rows, kBlock / lpg);
        switch (cpl) {
            case 1:
                if (blocks >= 4096) {  // four rows per lane group (as rms_norm)
                    hipLaunchKernelGGL((layer_norm_vec_kernel<1, false, kNormRpw>), dim3(ceil_div(blocks, kNormRpw)), dim3(kBlock), 0,
                                       stream, x, weight, bias, rows, dim, row_stride, eps_f, out);
                } else {
                    hipLaunchKernelGGL(layer_norm_vec_kernel<1>, dim3(blocks), dim3(kBlock), 0, stream, x, weight,
                                       bias, rows, dim, row_stride, eps_f, out);
                }
                break;
            case 2:
                hipLaunchKernelGGL(layer_norm_vec_kernel<2>, dim3(blocks), dim3(kBlock), 0, stream, x, weight, bias,
                                   rows, dim, row_stride, eps_f, out);
                break;
            default:
                hipLaunchKernelGGL(layer_norm_vec_kernel<4>, dim3(blocks), dim3(kBlock), 0, stream, x, weight, bias,
                                   rows, dim, row_stride, eps_f, out);
                break;
        }
        return launch_status("layer_norm");
    }
    const int64_t blocks = ceil_div(rows, kBlock / kWave);
    hipLaunchKernelGGL(layer_norm_scalar_kernel, dim3(blocks), dim3(kBlock), 0, stream, x, weight, bias, rows, dim,
                       row_stride, eps_f, out);
    return launch_status("layer_norm");
}

mlk_status mlk_layer_norm_bf16(const float* x, int64_t rows, int64_t dim, int64_t row_stride, const float* weight,
                               const float* bias, double eps, void* out, mlk_stream_t stream) {
    MLK_CHECK(rows >= 0 && dim >= 1, "x must have at least one dimension");
    const bool aligned = reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(weight) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(out) % 8 == 0 &&
                         (bias == nullptr || reinterpret_cast<uintptr_t>(bias) % 16 == 0) && row_stride % 4 == 0;
    const int64_t chunks = dim / 4;
    if (!aligned || dim % 4 != 0 || chunks > 64 || (chunks & (chunks - 1)) != 0) {
        set_error("layer_norm_bf16: rows without the vector form (use layer_norm)");
        return MLK_ERR_UNSUPPORTED;
    }
    if (rows == 0) return MLK_OK;
    MLK_CHECK(x != nullptr && weight != nullptr && out != nullptr, "null tensor pointer");
    const int64_t blocks = ceil_div(rows, kBlock / chunks);
    const double eps_f = static_cast<double>(static_cast<float>(eps));
    if (blocks >= 4096) {
        hipLaunchKernelGGL((layer_norm_vec_kernel<1, true, kNormRpw>), dim3(ceil_div(blocks, kNormRpw)), dim3(kBlock), 0, stream, x,
                           weight, bias, rows, dim, row_stride, eps_f, out);
    } else {
        hipLaunchKernelGGL((layer_norm_vec_kernel<1, true>), dim3(blocks), dim3(kBlock), 0, stream, x, weight, bias,
                           rows, dim, row_stride, eps_f, out);
    }
    return launch_status("layer_norm_bf16");
}

mlk_status mlk_swiglu(const float* x, int64_t rows, int64_t hidden, int64_t row_stride, float* out,
                      mlk_stream_t stream) {
    MLK_CHECK(rows >= 0 && hidden >= 1, "x must end in an even dimension [gate | up]");
    MLK_CHECK(rows == 0 || (x != nullptr && out != nullptr), "null tensor pointer");
    if (rows == 0) return MLK_OK;
    const int64_t blocks = ceil_div(rows * hidden, kBlock);
    if (rows * hidden < (int64_t{1} << 31)) {
        hipLaunchKernelGGL(swiglu_kernel<uint32_t>, dim3(blocks), dim3(kBlock), 0, stream, x, rows, hidden, row_stride,
                           out);
    } else {
        hipLaunchKernelGGL(swiglu_kernel<int64_t>, dim3(blocks), dim3(kBlock), 0, stream, x, rows, hidden, row_stride,
                           out);
    }
    return launch_status("swiglu");
}

}  // extern "C"
