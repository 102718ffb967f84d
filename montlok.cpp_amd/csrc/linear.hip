// Dense inference linear y = x W^T (+ bias) on the matrix cores.
//
// Stands in for linear_dispatch (rdt4quant_cpu/montlok.cpp:67-91), the
// oneDNN / at::linear call behind the `linear` op and every projection of
// mamba3_siso_layer, swiglu_mlp and mla_forward. x is fp32 [rows, K] with any
// row stride; W is [N, K] row-major in fp32 or bf16; y is fp32 with any row
// stride (so a projection can write into a column slice of a wider buffer).
//
// The projections of this model are skinny: K <= 512 and N <= ~1200 against
// tens of thousands of rows, i.e. ~70 flop per HBM byte, below the bf16 ridge.
// The kernel is laid out for that: x streams from HBM exactly once, W (a few
// hundred KB, L2 resident) is staged through LDS chunk by chunk.
//
//   block  = 4 waves, 64 rows (16 per wave); grid.y splits N only when there
//            are too few row blocks to fill the chip.
//   A      = the wave's 16 rows of x for one K chunk (256), loaded straight
//            from HBM into registers in the MFMA operand layout: lane l holds
//            row l%16, k = 8*(l/16) .. +7 of every 32-wide k step.
//   B      = a 64 x 256 chunk of W in LDS, read with one 16-byte LDS load per
//            lane per 16x16 tile.
//   MFMA   = bf16 weights: v_mfma_f32_16x16x32_bf16 with x rounded to bf16
//            (round to nearest even), fp32 accumulate; fp32 weights:
//            v_mfma_f32_16x16x4_f32, eight per 32-wide k step, fp32 throughout.
//   D      = lane l, register v holds row 4*(l/16)+v, column l%16 of a tile.
//
// K is reduced in an order of its own (the 8 k of a lane, then the four lane
// groups inside the MFMA); for fp32 weights the result differs from a
// sequential fp32 dot product by rounding only.

#include "mlk_common.h"

namespace mlk {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16;

constexpr int kRowsPerBlock = 64;
constexpr int kColsPerChunk = 64;
constexpr int kKChunk = 256;
constexpr int kSteps = kKChunk / 32;

template <bool BF16W>
struct WTraits;

template <>
struct WTraits<true> {
    using T = u16;
    static constexpr int kPitch = kKChunk + 8;  // +16 bytes per row: rows start on different banks
};

template <>
struct WTraits<false> {
    using T = float;
    static constexpr int kPitch = kKChunk + 4;
};

struct LinearArgs {
    const float* x;
    int64_t rows, K, x_stride;
    const void* w;
    const float* bias;
    int64_t N;
    float* out;
    int64_t out_stride;
};

__device__ __forceinline__ __bf16 bits_to_bf16(u16 v) { return __builtin_bit_cast(__bf16, v); }

// Loads 8 consecutive floats x[row, k .. k+7] (zero past K or past the last row).
template <bool VEC>
__device__ __forceinline__ void load_x8(const LinearArgs& p, int64_t row, int64_t k, float (&v)[8]) {
    if (row < p.rows && k + 8 <= p.K) {
        const float* src = p.x + row * p.x_stride + k;
        if constexpr (VEC) {
            const float4 lo = *reinterpret_cast<const float4*>(src);
            const float4 hi = *reinterpret_cast<const float4*>(src + 4);
            v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
            v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = src[j];
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v[j] = (row < p.rows && k + j < p.K) ? p.x[row * p.x_stride + k + j] : 0.0f;
        }
    }
}

// Copies W[n0 .. n0+63, k0 .. k0+255] into LDS, zero past N and K.
template <bool BF16W, bool VEC>
__device__ __forceinline__ void stage_w(const LinearArgs& p, int64_t n0, int64_t k0,
                                        typename WTraits<BF16W>::T* lds) {
    using T = typename WTraits<BF16W>::T;
    constexpr int kPitch = WTraits<BF16W>::kPitch;
    constexpr int kPerVec = 16 / sizeof(T);  // elements per 16-byte unit
    constexpr int kUnitsPerRow = kKChunk / kPerVec;
    const T* w = static_cast<const T*>(p.w);
    for (int u = threadIdx.x; u < kColsPerChunk * kUnitsPerRow; u += blockDim.x) {
        const int r = u / kUnitsPerRow;
        const int c = (u % kUnitsPerRow) * kPerVec;
        const int64_t n = n0 + r;
        const int64_t k = k0 + c;
        T* dst = lds + r * kPitch + c;
        if (VEC && n < p.N && k + kPerVec <= p.K) {
            *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(w + n * p.K + k);
        } else {
#pragma unroll
            for (int j = 0; j < kPerVec; ++j) dst[j] = (n < p.N && k + j < p.K) ? w[n * p.K + k + j] : T(0);
        }
    }
}

template <bool BF16W, bool VEC>
__global__ __launch_bounds__(256) void linear_kernel(LinearArgs p) {
    using T = typename WTraits<BF16W>::T;
    constexpr int kPitch = WTraits<BF16W>::kPitch;
    __shared__ __attribute__((aligned(16))) T w_lds[kColsPerChunk * kPitch];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col_in_tile = lane & 15;
    const int group = lane >> 4;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + 16 * wave;
    const int64_t my_row = row0 + col_in_tile;  // the A row this lane feeds
    const int64_t n_chunks = (p.N + kColsPerChunk - 1) / kColsPerChunk;
    const int64_t k_chunks = (p.K + kKChunk - 1) / kKChunk;

    // A operand for one K chunk: 8 k steps of 8 values per lane.
    bf16x8 a_bf[kSteps];
    float a_f[BF16W ? 1 : kSteps][8];

    auto load_a = [&](int64_t k0) {
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            float v[8];
            load_x8<VEC>(p, my_row, k0 + 32 * s + 8 * group, v);
            if constexpr (BF16W) {
#pragma unroll
                for (int j = 0; j < 8; ++j) a_bf[s][j] = static_cast<__bf16>(v[j]);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) a_f[s][j] = v[j];
            }
        }
    };

    if (k_chunks == 1) load_a(0);

    for (int64_t nc = blockIdx.y; nc < n_chunks; nc += gridDim.y) {
        const int64_t n0 = nc * kColsPerChunk;
        f32x4 acc[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

        for (int64_t kc = 0; kc < k_chunks; ++kc) {
            const int64_t k0 = kc * kKChunk;
            if (k_chunks > 1) load_a(k0);
            __syncthreads();  // previous chunk's readers are done with w_lds
            stage_w<BF16W, VEC>(p, n0, k0, w_lds);
            __syncthreads();
            const int steps = static_cast<int>((p.K - k0 + 31) / 32 < kSteps ? (p.K - k0 + 31) / 32 : kSteps);
#pragma unroll
            for (int s = 0; s < kSteps; ++s) {
                if (s < steps) {
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const T* src = w_lds + (16 * t + col_in_tile) * kPitch + 32 * s + 8 * group;
                        if constexpr (BF16W) {
                            const uint4 raw = *reinterpret_cast<const uint4*>(src);
                            const bf16x8 b = __builtin_bit_cast(bf16x8, raw);
                            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_bf[s], b, acc[t], 0, 0, 0);
                        } else {
                            const float4 b0 = *reinterpret_cast<const float4*>(src);
                            const float4 b1 = *reinterpret_cast<const float4*>(src + 4);
                            const float b[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
                            for (int j = 0; j < 8; ++j) {
                                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a_f[s][j], b[j], acc[t], 0, 0, 0);
                            }
                        }
                    }
                }
            }
        }

#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int64_t col = n0 + 16 * t + col_in_tile;
            if (col < p.N) {
                const float b = p.bias ? p.bias[col] : 0.0f;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int64_t row = row0 + 4 * group + v;
                    if (row < p.rows) p.out[row * p.out_stride + col] = acc[t][v] + b;
                }
            }
        }
    }
}

template <bool BF16W, bool VEC>
void launch(const LinearArgs& p, dim3 grid, hipStream_t stream) {
    hipLaunchKernelGGL((linear_kernel<BF16W, VEC>), grid, dim3(256), 0, stream, p);
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

}  // namespace
}  // namespace mlk

using namespace mlk;

extern "C" mlk_status mlk_linear(const float* x, int64_t rows, int64_t in_features, int64_t x_stride,
                                 const void* weight, int32_t weight_dtype, const float* bias, int64_t out_features,
                                 float* out, int64_t out_stride, mlk_stream_t stream) {
    MLK_CHECK(rows >= 0 && in_features > 0 && out_features > 0, "invalid linear geometry");
    MLK_CHECK(x_stride >= in_features, "x row stride must be at least in_features");
    MLK_CHECK(out_stride >= out_features, "out row stride must be at least out_features");
    MLK_CHECK(weight_dtype == MLK_DTYPE_F32 || weight_dtype == MLK_DTYPE_BF16, "weight dtype must be f32 or bf16");
    if (rows == 0) return MLK_OK;
    MLK_CHECK(x && weight && out, "null tensor pointer");
    LinearArgs p{x, rows, in_features, x_stride, weight, bias, out_features, out, out_stride};
    const int64_t row_blocks = ceil_div(rows, kRowsPerBlock);
    const int64_t n_chunks = ceil_div(out_features, kColsPerChunk);
    MLK_CHECK(row_blocks <= 0x7fffffff, "too many rows");
    // Split N over grid.y only while there are fewer than ~1024 blocks.
    int64_t gy = 1;
    while (gy < n_chunks && row_blocks * gy < 1024) ++gy;
    const dim3 grid(static_cast<unsigned>(row_blocks), static_cast<unsigned>(gy));
    const size_t wsize = weight_dtype == MLK_DTYPE_BF16 ? 2 : 4;
    const bool vec = aligned16(x) && x_stride % 4 == 0 && aligned16(weight) && (in_features * wsize) % 16 == 0;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (weight_dtype == MLK_DTYPE_BF16) {
        vec ? launch<true, true>(p, grid, s) : launch<true, false>(p, grid, s);
    } else {
        vec ? launch<false, true>(p, grid, s) : launch<false, false>(p, grid, s);
    }
    return launch_status("linear");
}
