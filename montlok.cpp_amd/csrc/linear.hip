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
//   block  = 8 waves, 128 rows (16 per wave); grid.y splits N only when there
//            are too few row blocks to fill the chip.
//   x      = the wave's 16 rows of x, loaded straight from HBM into registers
//            in the MFMA operand layout: lane l holds row l%16, k = 8*(l/16)
//            .. +7 of every 32-wide k step. With K within two chunks (512 for
//            bf16 weights, 256 for fp32) all of K stays in registers and x is
//            read once; beyond that (linear_kernel) it is reloaded per chunk.
//   B      = a 64-column chunk of W in LDS, double-buffered: the next chunk's
//            global loads are in flight while the MFMAs consume this one.
//            One 16-byte LDS load per lane per 16x16 tile.
//   MFMA   = bf16 weights: v_mfma_f32_16x16x32_bf16 with x rounded to bf16
//            (round to nearest even), fp32 accumulate; fp32 weights:
//            v_mfma_f32_16x16x4_f32, eight per 32-wide k step, fp32 throughout.
//   D      = lane l, register v holds row 4*(l/16)+v, column l%16 of a tile.
//
// Shapes with fewer 128-row blocks x 64-column chunks than CUs (a few
// thousand rows) take linear_small_kernel instead: one wave per 16 x 16
// output tile, operands straight from L2, no LDS.
//
// K is reduced in an order of its own (the 8 k of a lane, then the four lane
// groups inside the MFMA); for fp32 weights the result differs from a
// sequential fp32 dot product by rounding only.

#include <cstdlib>
#include <type_traits>
#include <cstring>

#include "mlk_common.h"
#include "tile_f32.h"

namespace mlk {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));  // the buffer builtins' 16-byte data type
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned short u16;

constexpr int kThreads = 512;                  // 8 waves
constexpr int kRowsPerBlock = 16 * (kThreads / 64);
constexpr int kColsPerChunk = 64;
constexpr int kBufferWord3 = 0x00020000;  // raw buffer resource, gfx9 data format fields

// Weight element type, K chunk staged per step, LDS row pitch (+16 bytes so
// consecutive rows start on different banks).
template <bool BF16W>
struct WTraits;
template <>
struct WTraits<true> {
    using T = u16;
    static constexpr int kKChunk = 256;
    static constexpr int kPitch = kKChunk + 8;
};
template <>
struct WTraits<false> {
    using T = float;
    static constexpr int kKChunk = 128;
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
    // Optional residual added to the result (out = residual + (x W^T + b),
    // the add as a separate fp32 rounding), rows res_stride apart.
    const float* residual;
    int64_t res_stride;
    // Optional grouped RMSNorm of x before the product (linear_small_kernel
    // only): weight and eps as the rms_norm operator takes them.
    const float* norm_w;
    double norm_eps;
};

// Loads 8 consecutive floats x[row, k .. k+7] (zero past K or past the last
// row). Rows past the end read the last row (in bounds) and are zeroed by the
// caller, so full-width loads need no branch around them.
template <bool VEC>
__device__ __forceinline__ void load_x8(const LinearArgs& p, int64_t row, int64_t k, float (&v)[8]) {
    if (k + 8 <= p.K) {
        const float* src = p.x + (row < p.rows ? row : p.rows - 1) * p.x_stride + k;
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

// A operand of one K chunk for the lane's row: step s holds k = k0 + 32s + 8g .. +7.
template <bool BF16W>
struct AFrag;
template <>
struct AFrag<true> {
    bf16x8 v[WTraits<true>::kKChunk / 32];
};
template <>
struct AFrag<false> {
    float v[WTraits<false>::kKChunk / 32][8];
};

template <bool BF16W, bool VEC>
__device__ __forceinline__ void load_a(const LinearArgs& p, int64_t row, int64_t k0, int group, int steps,
                                       AFrag<BF16W>& a) {
    constexpr int kSteps = WTraits<BF16W>::kKChunk / 32;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
        if (s < steps) {
            float v[8];
            load_x8<VEC>(p, row, k0 + 32 * s + 8 * group, v);
            const bool live = row < p.rows;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if constexpr (BF16W) {
                    a.v[s][j] = static_cast<__bf16>(live ? v[j] : 0.0f);
                } else {
                    a.v[s][j] = live ? v[j] : 0.0f;
                }
            }
        }
    }
}

// This thread's share of one W chunk W[n0 .. n0+63, k0 .. k0+kspan-1]: fixed
// 16-byte units, fetched into registers, later written to LDS (zero past N
// and K). Rows past N read row N - 1 (in bounds) and are zeroed at the store,
// so full-width fetches need no branch. Units at columns >= kspan are never
// read by the MFMA loop and skipped.
template <bool BF16W, bool VEC>
struct WStage {
    using T = typename WTraits<BF16W>::T;
    static constexpr int kPer = 16 / sizeof(T);
    static constexpr int kUnitsPerRow = WTraits<BF16W>::kKChunk / kPer;
    static constexpr int kUnits = (kColsPerChunk * kUnitsPerRow) / kThreads;
    uint4 reg[kUnits];

    // FULL (VEC, K a multiple of kPer): every unit is one 16-byte load with no branch around it (units past K
    // or past the chunk's span read a clamped address and are zeroed).
    template <bool FULL = false>
    __device__ __forceinline__ void fetch(const LinearArgs& p, int64_t n0, int64_t k0, int kspan) {
        const T* w = static_cast<const T*>(p.w);
#pragma unroll
        for (int u = 0; u < kUnits; ++u) {
            const int unit = threadIdx.x + u * kThreads;
            const int r = unit / kUnitsPerRow;
            const int c = (unit % kUnitsPerRow) * kPer;
            const int64_t n = n0 + r;
            const int64_t k = k0 + c;
            if constexpr (FULL) {
                // Every unit one 16-byte load from a clamped address, zeroed past K (K a multiple of kPer).
                const bool live = c < kspan && k < p.K;
                const uint4 v = *reinterpret_cast<const uint4*>(w + (n < p.N ? n : p.N - 1) * p.K + (live ? k : 0));
                reg[u] = live ? v : uint4{0u, 0u, 0u, 0u};
                continue;
            }
            if (c >= kspan) continue;
            if (VEC && k + kPer <= p.K) {
                reg[u] = *reinterpret_cast<const uint4*>(w + (n < p.N ? n : p.N - 1) * p.K + k);
            } else {
                T tmp[kPer];
#pragma unroll
                for (int j = 0; j < kPer; ++j) tmp[j] = (n < p.N && k + j < p.K) ? w[n * p.K + k + j] : T(0);
                reg[u] = __builtin_bit_cast(uint4, tmp);
            }
        }
    }

    __device__ __forceinline__ void store(const LinearArgs& p, int64_t n0, T* lds, int kspan) const {
#pragma unroll
        for (int u = 0; u < kUnits; ++u) {
            const int unit = threadIdx.x + u * kThreads;
            const int r = unit / kUnitsPerRow;
            const int c = (unit % kUnitsPerRow) * kPer;
            if (c < kspan) {
                *reinterpret_cast<uint4*>(lds + r * WTraits<BF16W>::kPitch + c) =
                    n0 + r < p.N ? reg[u] : uint4{0u, 0u, 0u, 0u};
            }
        }
    }
};

// Iterations run over (N chunk j of this block, K chunk kc), K fastest. W of
// iteration i+1 is fetched before the MFMAs of iteration i and written to the
// other LDS buffer after them: one barrier per iteration. When K spans several
// chunks, A is reloaded (from L2) at the start of each iteration.
// GS > 0 (fp32 weights, K = one chunk): the grouped RMSNorm of each row
// (groups of GS floats) applied to the loaded fragments first, the arithmetic
// of rms_norm_vec_kernel (tile_rms_norm), so the result equals rms_norm then
// this kernel bit for bit.
// BUF (no residual, output within 2 GiB): the results go out through a buffer resource, a store past its
// range dropped, so no store sits behind a branch: with the edge tests' branches the compiler cannot count
// the stores, and its wait for the next chunk's W loads (issued before them on the shared load/store
// counter) waited for every store of the chunk.
template <bool BF16W, bool VEC, bool MULTIK, int GS = 0, bool BUF = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(BUF ? 3 : 4, BUF ? 3 : 4))) void linear_kernel(LinearArgs p) {
    using T = typename WTraits<BF16W>::T;
    constexpr int KC = WTraits<BF16W>::kKChunk;
    constexpr int kSteps = KC / 32;
    constexpr int kPitch = WTraits<BF16W>::kPitch;
    __shared__ __attribute__((aligned(16))) T w_lds[2][kColsPerChunk * kPitch];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int li = lane & 15;
    const int group = lane >> 4;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + 16 * wave;
    const int64_t my_row = row0 + li;  // the A row this lane feeds
    const int64_t n_chunks = (p.N + kColsPerChunk - 1) / kColsPerChunk;
    const int64_t k_chunks = (p.K + KC - 1) / KC;
    const int64_t my_chunks = (n_chunks - blockIdx.y + gridDim.y - 1) / gridDim.y;
    const int64_t iters = my_chunks * k_chunks;
    if (iters <= 0) return;

    auto kspan_of = [&](int64_t kc) -> int {
        const int64_t rem = p.K - kc * KC;
        const int64_t span = ((rem < KC ? rem : KC) + 31) / 32 * 32;
        return static_cast<int>(span);
    };
    // One K chunk (!MULTIK): iteration = column chunk, no 64-bit division per iteration.
    auto n0_of = [&](int64_t it) { return (blockIdx.y + (MULTIK ? it / k_chunks : it) * gridDim.y) * kColsPerChunk; };

    WStage<BF16W, VEC> stage;
    AFrag<BF16W> a_cur;  // reloaded per iteration when K spans several chunks
    stage.template fetch<(GS > 0)>(p, n0_of(0), 0, kspan_of(0));
    load_a<BF16W, VEC>(p, my_row, 0, group, kspan_of(0) / 32, a_cur);
    if constexpr (GS > 0) {
        static_assert(!BF16W && !MULTIK, "the RMSNorm prologue needs all of K in fp32 fragments");
        float nw[kSteps][8];
        bool nlive[kSteps];
        tile_load8<kSteps>(p.norm_w, static_cast<int>(p.K), group, nw, nlive);
        tile_rms_norm<kSteps, GS>(a_cur.v, nw, p.norm_eps);
    }
    stage.store(p, n0_of(0), w_lds[0], kspan_of(0));
    __syncthreads();

    f32x4 acc[4];
    for (int64_t it = 0; it < iters; ++it) {
        const int64_t kc = MULTIK ? it % k_chunks : 0;
        const int64_t n0 = n0_of(it);
        const int steps = kspan_of(kc) / 32;
        const bool more = it + 1 < iters;
        const int64_t kc_next = MULTIK ? (it + 1) % k_chunks : 0;
        if constexpr (MULTIK) {
            if (it > 0) load_a<BF16W, VEC>(p, my_row, kc * KC, group, steps, a_cur);
        }
        // The bias before the next chunk's W: waiting for it then leaves the W loads in flight (loads and
        // stores retire in order on one counter).
        float bias[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // fetched with the chunk, used after its MFMAs
        if (p.bias != nullptr) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int64_t col = n0 + 16 * t + li;
                bias[t] = p.bias[col < p.N ? col : p.N - 1];
            }
        }
        // (FULL: fetched past the last chunk too, clamped rows that are never stored, so that no branch
        // separates these loads from the counter's view of the stores below.)
        if ((GS > 0) || more) stage.template fetch<(GS > 0)>(p, n0_of(it + 1), kc_next * KC, kspan_of(kc_next));
        if (kc == 0) {
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        const T* buf = w_lds[it & 1];
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            if (s < steps) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const T* src = buf + (16 * t + li) * kPitch + 32 * s + 8 * group;
                    if constexpr (BF16W) {
                        const bf16x8 b = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(src));
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_cur.v[s], b, acc[t], 0, 0, 0);
                    } else {
                        const float4 b0 = *reinterpret_cast<const float4*>(src);
                        const float4 b1 = *reinterpret_cast<const float4*>(src + 4);
                        const float b[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a_cur.v[s][j], b[j], acc[t], 0, 0, 0);
                        }
                    }
                }
            }
        }
        if constexpr (BUF) {
            static_assert(!MULTIK, "one K chunk: every iteration ends with its stores");
            const __amdgpu_buffer_rsrc_t out_rsrc = __builtin_amdgcn_make_buffer_rsrc(
                p.out, 0, static_cast<int>(((p.rows - 1) * p.out_stride + p.N) * 4), kBufferWord3);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int64_t col = n0 + 16 * t + li;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int64_t row = row0 + 4 * group + v;
                    const float y = acc[t][v] + bias[t];
                    const bool live = col < p.N && row < p.rows;
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y), out_rsrc,
                                                          live ? static_cast<uint32_t>((row * p.out_stride + col) * 4)
                                                               : 0x80000000u, 0, 0);
                }
            }
        } else if (kc == k_chunks - 1) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int64_t col = n0 + 16 * t + li;
                if (col < p.N) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int64_t row = row0 + 4 * group + v;
                        if (row < p.rows) {
                            const float y = acc[t][v] + bias[t];
                            p.out[row * p.out_stride + col] =
                                p.residual != nullptr ? p.residual[row * p.res_stride + col] + y : y;
                        }
                    }
                }
            }
        }
        if (more) stage.store(p, n0_of(it + 1), w_lds[(it + 1) & 1], kspan_of(kc_next));
        __syncthreads();
    }
}

// The tiled form for K within two chunks: each wave owns RT tiles of 16 rows
// (128 * RT rows per block) and holds its x fragments for all of K (KS
// chunks) in registers, so x is read once whatever N is, and every W fragment
// read from LDS feeds RT products. Iterations run over (N chunk, K chunk), W
// of the next one in flight as above. The products are formed transposed
// (W as the A operand, x as B; the same fragments the lanes hold above), so
// the accumulator of lane (g, l) holds row l, columns 4g .. 4g + 3 of a tile
// and leaves as one 16-byte store (scalar stores at a ragged N edge or an
// unaligned output).
// BUF > 0 (VEC, K a multiple of the 16-byte unit, N % 4 = 0, 16-byte aligned output and residual within
// 2 GiB): W fetched without per-unit branches (also past the last chunk, clamped) and the results stored
// through a buffer resource (a store past its range dropped), so no memory operation sits behind a branch
// and no wait covers the stores or the next W chunk. BUF = 1: no residual; BUF = 2: the residual fetched
// with the chunk's bias, before its W.
template <bool BF16W, bool VEC, int RT, int KS, int BUF = 0>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(RT * KS > 1 ? 2 : 4, RT * KS > 1 ? 2 : 4)))
void linear_tiles_kernel(LinearArgs p) {
    using T = typename WTraits<BF16W>::T;
    constexpr int KC = WTraits<BF16W>::kKChunk;
    constexpr int kSteps = KC / 32;
    constexpr int kPitch = WTraits<BF16W>::kPitch;
    __shared__ __attribute__((aligned(16))) T w_lds[2][kColsPerChunk * kPitch];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int li = lane & 15;
    const int group = lane >> 4;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * (kRowsPerBlock * RT) + 16 * RT * wave;
    const int64_t n_chunks = (p.N + kColsPerChunk - 1) / kColsPerChunk;
    const int64_t my_chunks = (n_chunks - blockIdx.y + gridDim.y - 1) / gridDim.y;
    if (my_chunks <= 0) return;
    const int64_t iters = my_chunks * KS;
    const bool vec_out = (reinterpret_cast<uintptr_t>(p.out) & 15) == 0 && p.out_stride % 4 == 0 &&
                         (p.residual == nullptr ||
                          ((reinterpret_cast<uintptr_t>(p.residual) & 15) == 0 && p.res_stride % 4 == 0));

    auto kspan_of = [&](int kc) -> int {
        const int64_t rem = p.K - static_cast<int64_t>(kc) * KC;
        const int64_t span = ((rem < KC ? rem : KC) + 31) / 32 * 32;
        return static_cast<int>(span);
    };
    auto n0_of = [&](int64_t it) { return (blockIdx.y + (it / KS) * gridDim.y) * kColsPerChunk; };

    WStage<BF16W, VEC> stage;
    AFrag<BF16W> a[RT][KS];
    stage.template fetch<(BUF > 0)>(p, n0_of(0), 0, kspan_of(0));
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int kc = 0; kc < KS; ++kc)
            load_a<BF16W, VEC>(p, row0 + 16 * rt + li, static_cast<int64_t>(kc) * KC, group, kspan_of(kc) / 32,
                               a[rt][kc]);
    stage.store(p, n0_of(0), w_lds[0], kspan_of(0));
    __syncthreads();

    f32x4 acc[RT][4];
    for (int64_t c = 0; c < my_chunks; ++c) {
        const int64_t n0 = n0_of(c * KS);
        f32x4 bias[4];  // columns n0 + 16t + 4g .. + 3
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int64_t col = n0 + 16 * t + 4 * group + v;
                bias[t][v] = p.bias != nullptr ? p.bias[col < p.N ? col : p.N - 1] : 0.0f;
            }
        }
        f32x4 resv[BUF == 2 ? RT : 1][4];  // BUF = 2: the residual of this chunk's outputs (clamped rows, columns)
        if constexpr (BUF == 2) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const int64_t row = row0 + 16 * rt + li;
                const float* rrow = p.residual + (row < p.rows ? row : p.rows - 1) * p.res_stride;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int64_t col = n0 + 16 * t + 4 * group;
                    resv[rt][t] = *reinterpret_cast<const f32x4*>(rrow + (col < p.N ? col : p.N - 4));
                }
            }
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[rt][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kc = 0; kc < KS; ++kc) {
            const int64_t it = c * KS + kc;
            const bool more = it + 1 < iters;
            const int kc_next = (kc + 1) % KS;
            if (BUF > 0 || more) stage.template fetch<(BUF > 0)>(p, n0_of(it + 1), static_cast<int64_t>(kc_next) * KC, kspan_of(kc_next));
            const int steps = kspan_of(kc) / 32;
            const T* buf = w_lds[it & 1];
#pragma unroll
            for (int s = 0; s < kSteps; ++s) {
                if (s < steps) {
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const T* src = buf + (16 * t + li) * kPitch + 32 * s + 8 * group;
                        if constexpr (BF16W) {
                            const bf16x8 bv = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(src));
#pragma unroll
                            for (int rt = 0; rt < RT; ++rt)
                                acc[rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bv, a[rt][kc].v[s], acc[rt][t], 0, 0, 0);
                        } else {
                            const float4 b0 = *reinterpret_cast<const float4*>(src);
                            const float4 b1 = *reinterpret_cast<const float4*>(src + 4);
                            const float bv[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
                            for (int j = 0; j < 8; ++j)
#pragma unroll
                                for (int rt = 0; rt < RT; ++rt)
                                    acc[rt][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(bv[j], a[rt][kc].v[s][j], acc[rt][t], 0, 0, 0);
                        }
                    }
                }
            }
            if (BUF > 0 && kc == KS - 1) {
                const __amdgpu_buffer_rsrc_t out_rsrc = __builtin_amdgcn_make_buffer_rsrc(
                    p.out, 0, static_cast<int>(((p.rows - 1) * p.out_stride + p.N) * 4), kBufferWord3);
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    const int64_t row = row0 + 16 * rt + li;
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const int64_t col = n0 + 16 * t + 4 * group;
                        f32x4 y = acc[rt][t] + bias[t];
                        if constexpr (BUF == 2) y = resv[rt][BUF == 2 ? t : 0] + y;
                        const bool live = row < p.rows && col < p.N;
                        __builtin_amdgcn_raw_buffer_store_b128(
                            __builtin_bit_cast(u32x4, y), out_rsrc,
                            live ? static_cast<uint32_t>((row * p.out_stride + col) * 4) : 0x80000000u, 0, 0);
                    }
                }
            } else if (kc == KS - 1) {
                const bool full = vec_out && n0 + kColsPerChunk <= p.N;
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    const int64_t row = row0 + 16 * rt + li;
                    if (row < p.rows) {
                        float* orow = p.out + row * p.out_stride + n0 + 4 * group;
                        const float* rrow = p.residual != nullptr ? p.residual + row * p.res_stride + n0 + 4 * group : nullptr;
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            f32x4 y = acc[rt][t] + bias[t];
                            if (full) {
                                if (p.residual != nullptr) y = *reinterpret_cast<const f32x4*>(rrow + 16 * t) + y;
                                *reinterpret_cast<f32x4*>(orow + 16 * t) = y;
                            } else {
#pragma unroll
                                for (int v = 0; v < 4; ++v) {
                                    if (n0 + 16 * t + 4 * group + v < p.N) {
                                        orow[16 * t + v] = p.residual != nullptr ? rrow[16 * t + v] + y[v] : y[v];
                                    }
                                }
                            }
                        }
                    }
                }
            }
            if (more) stage.store(p, n0_of(it + 1), w_lds[(it + 1) & 1], kspan_of(kc_next));
            __syncthreads();
        }
    }
}

// The small-problem form, for shapes whose 128-row blocks cannot fill the
// chip (a few thousand rows): one wave per 16 x 16 output tile, so the grid
// has rows/16 x N/16 waves. Both operands come straight from memory (L2) in
// the MFMA fragment layout, every load of the tile issued before the first
// product, no LDS and no barrier. KS 32-wide k steps are held in registers
// (K <= 32 KS, K a multiple of 8: an 8-wide segment lies wholly inside or
// wholly past K, and segments past K read column 0 and are zeroed). As in the
// tiled form the products are transposed (W as the A operand), leaving lane
// (g, l) with row l, columns 4g .. 4g + 3. fp32 weights accumulate the even
// and odd k of each lane in two chains, summed at the end.
//
// GS > 0 applies the grouped RMSNorm of x (groups of GS floats, GS in 8, 16,
// 32, 64) to the loaded fragments first, with the arithmetic of
// rms_norm_vec_kernel: per 4-float chunk the fp64 partial (a^2 + b^2) +
// (c^2 + d^2), the group's chunks combined by the same butterfly (chunk c of
// the group is lane (c / 2) % 4's half c % 2 of its segment, so the levels
// are: the two steps of a 64-group in registers, lanes 32 apart, lanes 16
// apart, the two halves in registers), scale = 1 / sqrt(sum / GS + eps),
// x * scale * w rounded once. The normalised x is bit-identical to the
// rms_norm operator's output, so the product is that of rms_norm then linear.
template <bool BF16W, int KS, int GS, bool ALL_LIVE = false>
__global__ __launch_bounds__(64) void linear_small_kernel(LinearArgs p) {
    const int lane = threadIdx.x;
    const int li = lane & 15;
    const int group = lane >> 4;
    const int64_t n_tiles = (p.N + 15) / 16;
    // Tile order: consecutive blocks go to the 8 XCDs in turn, so XCD x takes the x-th eighth of the tiles
    // (whole row tiles together): a row tile's x rows are fetched into one L2 for all its column tiles, and
    // rows a producer kernel wrote from the same XCD (the Mamba mixer places windows this way) are L2 hits.
    unsigned lin = blockIdx.x;
    if (gridDim.x % 8 == 0) lin = (lin % 8) * (gridDim.x / 8) + lin / 8;
    const int64_t row0 = static_cast<int64_t>(lin / n_tiles) * 16;
    const int64_t n0 = static_cast<int64_t>(lin % n_tiles) * 16;
    const int64_t xr = row0 + li < p.rows ? row0 + li : p.rows - 1;
    const int64_t wr = n0 + li < p.N ? n0 + li : p.N - 1;
    const int K = static_cast<int>(p.K);
    float xv[KS][8];
    bool live[KS];
    tile_load8<KS>(p.x + xr * p.x_stride, K, group, xv, live);
    if constexpr (GS > 0) {
        float nw[KS][8];
        bool nlive[KS];
        tile_load8<KS>(p.norm_w, K, group, nw, nlive);
        tile_rms_norm<KS, GS>(xv, nw, p.norm_eps);
    }
    f32x4 bias = {0.0f, 0.0f, 0.0f, 0.0f};
    if (p.bias != nullptr) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int64_t col = n0 + 4 * group + v;
            bias[v] = p.bias[col < p.N ? col : p.N - 1];
        }
    }
    // The 16-byte epilogue's residual values are fetched with the operands (this lane's row, clamped), so
    // their latency passes behind the products instead of after them.
    const bool vec_out = (reinterpret_cast<uintptr_t>(p.out) & 15) == 0 && p.out_stride % 4 == 0 && n0 + 16 <= p.N &&
                         (p.residual == nullptr ||
                          ((reinterpret_cast<uintptr_t>(p.residual) & 15) == 0 && p.res_stride % 4 == 0));
    f32x4 resv = {0.0f, 0.0f, 0.0f, 0.0f};
    if (vec_out && p.residual != nullptr) resv = *reinterpret_cast<const f32x4*>(p.residual + xr * p.res_stride + n0 + 4 * group);
    f32x4 y;
    if constexpr (BF16W) {
        const u16* wrow = static_cast<const u16*>(p.w) + wr * p.K;
        uint4 wv[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const int k = 32 * s + 8 * group;
            wv[s] = *reinterpret_cast<const uint4*>(wrow + (live[s] ? k : 0));
        }
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            bf16x8 a;
            bf16x8 b = __builtin_bit_cast(bf16x8, live[s] ? wv[s] : uint4{0u, 0u, 0u, 0u});
#pragma unroll
            for (int j = 0; j < 8; ++j) a[j] = static_cast<__bf16>(live[s] ? xv[s][j] : 0.0f);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b, a, acc, 0, 0, 0);
        }
        y = acc;
    } else {
        float wv[KS][8];
        bool wlive[KS];
        tile_load8<KS>(static_cast<const float*>(p.w) + wr * p.K, K, group, wv, wlive);
        y = tile_mfma_f32<KS, ALL_LIVE>(wv, xv, live);
    }
    y += bias;
    const int64_t row = row0 + li;
    if (row < p.rows) {
        float* dst = p.out + row * p.out_stride + n0 + 4 * group;
        const float* res = p.residual != nullptr ? p.residual + row * p.res_stride + n0 + 4 * group : nullptr;
        if (vec_out) {
            if (res != nullptr) y = resv + y;
            *reinterpret_cast<f32x4*>(dst) = y;
        } else {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                if (n0 + 4 * group + v < p.N) dst[v] = res != nullptr ? res[v] + y[v] : y[v];
            }
        }
    }
}

template <bool BF16W, int KS, int GS = 0>
void launch_small(const LinearArgs& p, int64_t tiles, hipStream_t stream) {
    // fp32 weights with K filling all KS steps skip the per-operand selects.
    if (!BF16W && p.K == 32 * KS) {
        hipLaunchKernelGGL((linear_small_kernel<BF16W, KS, GS, true>), dim3(static_cast<unsigned>(tiles)), dim3(64),
                           0, stream, p);
        return;
    }
    hipLaunchKernelGGL((linear_small_kernel<BF16W, KS, GS>), dim3(static_cast<unsigned>(tiles)), dim3(64), 0, stream,
                       p);
}

// The small form with the RMSNorm prologue: K steps by K, group size by gs.
template <bool BF16W, int GS>
void launch_small_norm(const LinearArgs& p, int64_t tiles, hipStream_t stream) {
    if (p.K <= 64) {
        launch_small<BF16W, 2, GS>(p, tiles, stream);
    } else if (p.K <= 128) {
        launch_small<BF16W, 4, GS>(p, tiles, stream);
    } else {
        launch_small<BF16W, 8, GS>(p, tiles, stream);
    }
}

// bf16 weights with K <= 256 on the 32 x 32 x 16 matrix cores: each wave owns
// 32 rows (256 per block), holds their bf16 x fragments for all of K, and
// each W fragment read from LDS (32 columns x 16 k) feeds a 32-row product,
// half the LDS traffic per row of the 16 x 16 x 32 form. Operands transposed
// as in the tiled form (W as A, x as B): lane (h, l) of the accumulator holds
// row l, columns 8j + 4h .. + 3 (j = 0..3) of a 32-column tile. W chunks of 64
// columns are staged and double-buffered as in the other forms.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void linear_t32_kernel(LinearArgs p) {
    using T = u16;
    constexpr int KC = WTraits<true>::kKChunk;  // 256: all of K
    constexpr int kPitch = WTraits<true>::kPitch;
    constexpr int kSteps = KC / 16;
    __shared__ __attribute__((aligned(16))) T w_lds[2][kColsPerChunk * kPitch];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r32 = lane & 31;
    const int h = lane >> 5;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * (2 * kRowsPerBlock) + 32 * wave;
    const int64_t n_chunks = (p.N + kColsPerChunk - 1) / kColsPerChunk;
    const int64_t my_chunks = (n_chunks - blockIdx.y + gridDim.y - 1) / gridDim.y;
    if (my_chunks <= 0) return;
    const int kspan = static_cast<int>((p.K + 31) / 32 * 32);
    const bool vec_out = (reinterpret_cast<uintptr_t>(p.out) & 15) == 0 && p.out_stride % 4 == 0 &&
                         (p.residual == nullptr ||
                          ((reinterpret_cast<uintptr_t>(p.residual) & 15) == 0 && p.res_stride % 4 == 0));
    auto n0_of = [&](int64_t c) { return (blockIdx.y + c * gridDim.y) * kColsPerChunk; };

    WStage<true, VEC> stage;
    stage.fetch(p, n0_of(0), 0, kspan);
    // x fragments: step s holds row r32's k = 16 s + 8 h .. + 7 (zero past K or past the rows).
    bf16x8 xf[kSteps];
    {
        const int64_t row = row0 + r32;
        const bool live_row = row < p.rows;
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            float v[8];
            load_x8<VEC>(p, row, 16 * s + 8 * h, v);
#pragma unroll
            for (int j = 0; j < 8; ++j) xf[s][j] = static_cast<__bf16>(live_row ? v[j] : 0.0f);
        }
    }
    stage.store(p, n0_of(0), w_lds[0], kspan);
    __syncthreads();

    for (int64_t c = 0; c < my_chunks; ++c) {
        const int64_t n0 = n0_of(c);
        const bool more = c + 1 < my_chunks;
        if (more) stage.fetch(p, n0_of(c + 1), 0, kspan);
        const T* buf = w_lds[c & 1];
        f32x16 acc[2];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[t][v] = 0.0f;
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            if (16 * s < kspan) {
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const bf16x8 wv = __builtin_bit_cast(
                        bf16x8, *reinterpret_cast<const uint4*>(buf + (32 * t + r32) * kPitch + 16 * s + 8 * h));
                    acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wv, xf[s], acc[t], 0, 0, 0);
                }
            }
        }
        const int64_t row = row0 + r32;
        if (row < p.rows) {
            float* orow = p.out + row * p.out_stride;
            const float* rrow = p.residual != nullptr ? p.residual + row * p.res_stride : nullptr;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int64_t col = n0 + 32 * t + 8 * j + 4 * h;
                    f32x4 y = {acc[t][4 * j], acc[t][4 * j + 1], acc[t][4 * j + 2], acc[t][4 * j + 3]};
                    if (p.bias != nullptr) {
#pragma unroll
                        for (int u = 0; u < 4; ++u) y[u] += p.bias[col + u < p.N ? col + u : p.N - 1];
                    }
                    if (col + 4 <= p.N && vec_out) {
                        if (rrow != nullptr) y = *reinterpret_cast<const f32x4*>(rrow + col) + y;
                        *reinterpret_cast<f32x4*>(orow + col) = y;
                    } else {
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            if (col + u < p.N) orow[col + u] = rrow != nullptr ? rrow[col + u] + y[u] : y[u];
                        }
                    }
                }
        }
        if (more) stage.store(p, n0_of(c + 1), w_lds[(c + 1) & 1], kspan);
        __syncthreads();
    }
}

// bf16 weights, K = 256 and a wide output, streaming form: the weights stay in
// registers and x streams through LDS. Each wave owns 32 columns of W (its A
// fragments for all of K: 16 k steps x 16 bytes per lane), a block of 8 waves
// a group of 256 columns. Blocks are persistent, one per CU: block (row part,
// column group) walks its row part's 32-row tiles; each x tile is loaded from
// HBM into registers a tile ahead, rounded to bf16 and written to one of two
// LDS buffers (one barrier per tile). The column groups of a row part run on
// one XCD (round-robin dispatch puts block i on XCD i % 8), so x comes from
// HBM once and from that XCD's L2 for the other groups (without that
// placement: 643 instead of 455 us). Per 32 x 32 tile the chain over k is
// linear_t32_kernel's (32 x 32 x 16 MFMA, W as A, x as B, k steps in order),
// so the two kernels give the same bits; the W fragments are read once per
// block instead of from LDS once per 64 columns and 256 rows. Accumulator lane
// (h, l): row l, columns 8j + 4h .. + 3 (j = 0..3), stored as 16-byte pieces.
//   262144 x 256 -> 1192: 455 us against 508-528 us for linear_t32_kernel.
//   Measured and not kept: two 32-row chains per wave (515 us), the output
//   rows staged through LDS so each store writes whole 128-byte pieces (459
//   us), non-temporal stores (1.5 ms), x two tiles ahead (469 us). Without
//   its stores the kernel takes 261 us, and a plain fill writes the 1.25 GB
//   output in 187 us: the stores add their whole time to the rest, which is
//   what linear_stream_sw_kernel below works on: 445 us (and then
//   linear_stream_io_kernel, the default: 361 us).
constexpr int kStreamWaves = 8;
constexpr int kStreamCols = 32 * kStreamWaves;  // columns per block
constexpr int kStreamRT = 1;                    // 32-row tiles per step
constexpr int kStreamRows = 32 * kStreamRT;     // rows per step
constexpr int kStreamK = 256;                   // the form takes K = 256 exactly (16-byte aligned operands)

// BUF: no bias or residual, N % 4 = 0, 16-byte aligned output within 2 GiB: the results go out through a
// buffer resource, a store past its range dropped, so no store sits behind a branch. With the edge tests'
// branches the compiler cannot count the stores, and its wait for the next tile's x loads (issued before
// them on the shared load/store counter) waited for every store of the tile.
template <int K, bool BUF = false>
__global__ __launch_bounds__(64 * kStreamWaves) __attribute__((amdgpu_waves_per_eu(2, 2)))
void linear_stream_kernel(LinearArgs p, int col_groups, int row_parts) {
    using T = u16;
    constexpr int kSteps = K / 16;
    constexpr int kPitch = K + 8;             // LDS row pitch in bf16 (+16 bytes)
    constexpr int kThr = 64 * kStreamWaves;
    constexpr int kTPR = kThr / kStreamRows;  // threads per x row
    constexpr int kXPer = K / kTPR;           // x floats per thread per tile
    // x fragments read from LDS a part of K at a time (K = 512: a quarter, so that the W fragments, 128
    // registers, the next tile's x and the part fit two waves per SIMD); the products keep the order of k.
    constexpr int kXParts = K / 128;
    static_assert(kSteps % kXParts == 0, "whole parts of K");
    static_assert(kXPer % 8 == 0, "whole 16-byte bf16 units per thread");
    __shared__ __attribute__((aligned(16))) T x_lds[2][kStreamRows * kPitch];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r32 = lane & 31;
    const int h = lane >> 5;
    // Block -> (XCD, local index) -> (row part, column group): the groups of a row part share an XCD.
    const int xcd = blockIdx.x % 8;
    const int local = blockIdx.x / 8;
    const int cg = local % col_groups;
    const int rpl = local / col_groups;
    const int rp = rpl * 8 + xcd;
    if (rp >= row_parts) return;
    const int64_t tiles = (p.rows + kStreamRows - 1) / kStreamRows;
    const int64_t t_begin = tiles * rp / row_parts, t_end = tiles * (rp + 1) / row_parts;
    if (t_begin >= t_end) return;
    const int64_t n_wave = static_cast<int64_t>(cg) * kStreamCols + 32 * wave;  // this wave's first column
    const bool wave_live = n_wave < p.N;
    const bool vec_out = (reinterpret_cast<uintptr_t>(p.out) & 15) == 0 && p.out_stride % 4 == 0 &&
                         (p.residual == nullptr ||
                          ((reinterpret_cast<uintptr_t>(p.residual) & 15) == 0 && p.res_stride % 4 == 0));

    // W fragments: step s holds column n_wave + r32, k = 16 s + 8 h .. + 7 (zero past N).
    uint4 wf[kSteps];
    {
        const T* w = static_cast<const T*>(p.w);
        const int64_t n = n_wave + r32;
        const T* wrow = w + (n < p.N ? n : p.N - 1) * K + 8 * h;
        const uint32_t keep = n < p.N ? 0xffffffffu : 0u;
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const uint4 v = *reinterpret_cast<const uint4*>(wrow + 16 * s);
            wf[s] = uint4{v.x & keep, v.y & keep, v.z & keep, v.w & keep};
        }
    }
    // x tile loads: thread t takes row t / kTPR, columns kXPer (t % kTPR) .. (rows past the end read the
    // last row and are zeroed where they are converted).
    const int xr = threadIdx.x / kTPR, xc = kXPer * (threadIdx.x % kTPR);
    float4 xv[kXPer / 4];
    auto load_tile = [&](int64_t t) {
        const int64_t row = t * kStreamRows + xr;
        const float* src = p.x + (row < p.rows ? row : p.rows - 1) * p.x_stride + xc;
#pragma unroll
        for (int q = 0; q < kXPer / 4; ++q) xv[q] = *reinterpret_cast<const float4*>(src + 4 * q);
    };
    auto store_tile = [&](int64_t t, T* buf) {
        const bool live = t * kStreamRows + xr < p.rows;
#pragma unroll
        for (int u = 0; u < kXPer / 8; ++u) {
            const float4 a = xv[2 * u], b = xv[2 * u + 1];
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            bf16x8 o;
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = static_cast<__bf16>(live ? v[j] : 0.0f);
            *reinterpret_cast<bf16x8*>(buf + xr * kPitch + xc + 8 * u) = o;
        }
    };

    load_tile(t_begin);
    store_tile(t_begin, x_lds[0]);
    __syncthreads();
    auto iteration = [&](int64_t t, auto par_c) {
        constexpr int PAR = decltype(par_c)::value;  // (t - t_begin) % 2: the LDS buffer of tile t
        const bool more = t + 1 < t_end;
        if (more) load_tile(t + 1);
        const T* buf = x_lds[PAR];
        f32x16 acc[kStreamRT];
#pragma unroll
        for (int m = 0; m < kStreamRT; ++m)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[m][v] = 0.0f;
        if (wave_live) {
#pragma unroll
            for (int part = 0; part < kXParts; ++part) {
                constexpr int kPS = kSteps / kXParts;
                uint4 xb[kStreamRT][kPS];
#pragma unroll
                for (int s = 0; s < kPS; ++s)
#pragma unroll
                    for (int m = 0; m < kStreamRT; ++m)
                        xb[m][s] = *reinterpret_cast<const uint4*>(buf + (32 * m + r32) * kPitch + 16 * (part * kPS + s) + 8 * h);
#pragma unroll
                for (int s = 0; s < kPS; ++s) {
#pragma unroll
                    for (int m = 0; m < kStreamRT; ++m) {
                        acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, wf[part * kPS + s]),
                                                                         __builtin_bit_cast(bf16x8, xb[m][s]), acc[m], 0,
                                                                         0, 0);
                    }
                }
            }
            if constexpr (!BUF) {
#pragma unroll
            for (int m = 0; m < kStreamRT; ++m) {
                const int64_t row = t * kStreamRows + 32 * m + r32;
                if (row < p.rows) {
                    float* orow = p.out + row * p.out_stride;
                    const float* rrow = p.residual != nullptr ? p.residual + row * p.res_stride : nullptr;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int64_t col = n_wave + 8 * j + 4 * h;
                        f32x4 y = {acc[m][4 * j], acc[m][4 * j + 1], acc[m][4 * j + 2], acc[m][4 * j + 3]};
                        if (p.bias != nullptr) {
#pragma unroll
                            for (int u = 0; u < 4; ++u) y[u] += p.bias[col + u < p.N ? col + u : p.N - 1];
                        }
                        if (col + 4 <= p.N && vec_out) {
                            if (rrow != nullptr) y = *reinterpret_cast<const f32x4*>(rrow + col) + y;
                            *reinterpret_cast<f32x4*>(orow + col) = y;
                        } else {
#pragma unroll
                            for (int u = 0; u < 4; ++u) {
                                if (col + u < p.N) orow[col + u] = rrow != nullptr ? rrow[col + u] + y[u] : y[u];
                            }
                        }
                    }
                }
            }
            }
        }
        if constexpr (BUF) {  // every wave, outside any branch (a wave past N stores nothing)
            const __amdgpu_buffer_rsrc_t out_rsrc = __builtin_amdgcn_make_buffer_rsrc(
                p.out, 0, static_cast<int>(((p.rows - 1) * p.out_stride + p.N) * 4), kBufferWord3);
#pragma unroll
            for (int m = 0; m < kStreamRT; ++m) {
                const int64_t row = t * kStreamRows + 32 * m + r32;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int64_t col = n_wave + 8 * j + 4 * h;
                    const f32x4 y = {acc[m][4 * j], acc[m][4 * j + 1], acc[m][4 * j + 2], acc[m][4 * j + 3]};
                    const bool live = row < p.rows && col < p.N;
                    const uint32_t off = live ? static_cast<uint32_t>((row * p.out_stride + col) * 4) : 0x80000000u;
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, y), out_rsrc, off, 0, 0);
                }
            }
        }
        if (more) store_tile(t + 1, x_lds[PAR ^ 1]);
        __syncthreads();
    };
    for (int64_t t = t_begin; t < t_end; t += 2) {
        iteration(t, std::integral_constant<int, 0>{});
        if (t + 1 < t_end) iteration(t + 1, std::integral_constant<int, 1>{});
    }
}

// The streaming form with its output stores on separate waves: waves 0..7
// compute as in linear_stream_kernel but leave each 32 x 256 result tile in
// one of two LDS buffers; waves 8..11 store the tile of the previous step from
// there (whole 1 KB row pieces per instruction), so the global stores run
// while the next tile's products are formed. Same products and order as
// linear_stream_kernel (and linear_t32_kernel), same bits. 12 waves put three
// on a SIMD: the computing waves load x's fragments half of K at a time and
// the storing waves unroll by two, which keeps both within 168 registers
// without spills. 262144 x 256 -> 1192: 445 us against 457 us for
// linear_stream_kernel. Where linear_stream_io_kernel takes the shape it is the
// default; MLK_LINEAR_STORE_WAVES=sw selects this form, =0 linear_stream_kernel.
// Its stores sit behind branches (the output edge tests), so the compiler's
// shared load/store counter makes each step's x load wait for the previous
// step's stores: the IO-wave form's buffer stores remove that.
constexpr int kStoreWaves = 4;

__global__ __launch_bounds__(64 * (kStreamWaves + kStoreWaves))
void linear_stream_sw_kernel(LinearArgs p, int col_groups, int row_parts) {
    using T = u16;
    constexpr int kSteps = kStreamK / 16;
    constexpr int kPitch = kStreamK + 8;      // x tile row pitch in bf16 (+16 bytes)
    constexpr int kOPitch = kStreamCols + 4;  // output tile row pitch in floats (+16 bytes)
    constexpr int kThr = 64 * kStreamWaves;   // the computing waves' threads
    constexpr int kTPR = kThr / kStreamRows;  // threads per x row
    constexpr int kXPer = kStreamK / kTPR;    // x floats per thread per tile
    static_assert(kStreamRT == 1 && kXPer % 8 == 0, "one 32-row tile per step, whole 16-byte bf16 units");
    __shared__ __attribute__((aligned(16))) T x_lds[2][kStreamRows * kPitch];
    __shared__ __attribute__((aligned(16))) float o_lds[2][kStreamRows * kOPitch];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool storer = wave >= kStreamWaves;
    const int r32 = lane & 31;
    const int h = lane >> 5;
    const int xcd = blockIdx.x % 8;
    const int local = blockIdx.x / 8;
    const int cg = local % col_groups;
    const int rpl = local / col_groups;
    const int rp = rpl * 8 + xcd;
    if (rp >= row_parts) return;
    const int64_t tiles = (p.rows + kStreamRows - 1) / kStreamRows;
    const int64_t t_begin = tiles * rp / row_parts, t_end = tiles * (rp + 1) / row_parts;
    if (t_begin >= t_end) return;
    const int64_t n_block = static_cast<int64_t>(cg) * kStreamCols;
    const int64_t n_wave = n_block + 32 * (storer ? 0 : wave);  // a computing wave's first column
    const bool wave_live = !storer && n_wave < p.N;
    const bool vec_out = (reinterpret_cast<uintptr_t>(p.out) & 15) == 0 && p.out_stride % 4 == 0 &&
                         (p.residual == nullptr ||
                          ((reinterpret_cast<uintptr_t>(p.residual) & 15) == 0 && p.res_stride % 4 == 0));

    uint4 wf[kSteps];
    if (!storer) {  // the storing waves hold no weights
        const T* w = static_cast<const T*>(p.w);
        const int64_t n = n_wave + r32;
        const T* wrow = w + (n < p.N ? n : p.N - 1) * kStreamK + 8 * h;
        const uint32_t keep = n < p.N ? 0xffffffffu : 0u;
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const uint4 v = *reinterpret_cast<const uint4*>(wrow + 16 * s);
            wf[s] = uint4{v.x & keep, v.y & keep, v.z & keep, v.w & keep};
        }
    }
    const int xr = threadIdx.x / kTPR, xc = kXPer * (threadIdx.x % kTPR);
    float4 xv[kXPer / 4];
    auto load_tile = [&](int64_t t) {
        const int64_t row = t * kStreamRows + xr;
        const float* src = p.x + (row < p.rows ? row : p.rows - 1) * p.x_stride + xc;
#pragma unroll
        for (int q = 0; q < kXPer / 4; ++q) xv[q] = *reinterpret_cast<const float4*>(src + 4 * q);
    };
    auto store_tile = [&](int64_t t, T* buf) {
        const bool live = t * kStreamRows + xr < p.rows;
#pragma unroll
        for (int u = 0; u < kXPer / 8; ++u) {
            const float4 a = xv[2 * u], b = xv[2 * u + 1];
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            bf16x8 o;
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = static_cast<__bf16>(live ? v[j] : 0.0f);
            *reinterpret_cast<bf16x8*>(buf + xr * kPitch + xc + 8 * u) = o;
        }
    };
    // The storing waves: tile t of buffer `buf`, lane u = 64 (wave - 8) + lane takes float4 u + 256 i of the
    // tile (row (u + 256 i) / 64, columns 4 ((u + 256 i) % 64) ..), so each instruction writes one row's
    // 1 KB of this column group.
    auto write_out = [&](int64_t t, const float* buf) __attribute__((always_inline)) {
        const int u = 64 * (wave - kStreamWaves) + lane;
#pragma unroll 2
        for (int i = 0; i < kStreamRows * kStreamCols / 4 / (64 * kStoreWaves); ++i) {
            const int e = u + 64 * kStoreWaves * i;
            const int rr = e / (kStreamCols / 4), c4 = 4 * (e % (kStreamCols / 4));
            const int64_t row = t * kStreamRows + rr;
            const int64_t col = n_block + c4;
            if (row >= p.rows || col >= p.N) continue;
            f32x4 y = *reinterpret_cast<const f32x4*>(buf + rr * kOPitch + c4);
            float* orow = p.out + row * p.out_stride;
            const float* rrow = p.residual != nullptr ? p.residual + row * p.res_stride : nullptr;
            if (p.bias != nullptr) {
#pragma unroll
                for (int q = 0; q < 4; ++q) y[q] += p.bias[col + q < p.N ? col + q : p.N - 1];
            }
            if (col + 4 <= p.N && vec_out) {
                if (rrow != nullptr) y = *reinterpret_cast<const f32x4*>(rrow + col) + y;
                *reinterpret_cast<f32x4*>(orow + col) = y;
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if (col + q < p.N) orow[col + q] = rrow != nullptr ? rrow[col + q] + y[q] : y[q];
                }
            }
        }
    };

    // Both kinds of wave pass the same barriers: one before the first step and one after each step.
    if (storer) {
        __syncthreads();
        for (int64_t t = t_begin; t < t_end; ++t) {
            if (t > t_begin) write_out(t - 1, o_lds[(t - 1 - t_begin) & 1]);
            __syncthreads();
        }
        write_out(t_end - 1, o_lds[(t_end - 1 - t_begin) & 1]);
        return;
    }
    load_tile(t_begin);
    store_tile(t_begin, x_lds[0]);
    __syncthreads();
    auto iteration = [&](int64_t t, auto par_c) {
        constexpr int PAR = decltype(par_c)::value;  // (t - t_begin) % 2: the buffers of tile t
        const bool more = t + 1 < t_end;
        if (more) load_tile(t + 1);
        if (wave_live) {
            const T* buf = x_lds[PAR];
            f32x16 acc;
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
            // x fragments in two halves of K: within the registers of three waves per SIMD.
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                uint4 xb[kSteps / 2];
#pragma unroll
                for (int s = 0; s < kSteps / 2; ++s)
                    xb[s] = *reinterpret_cast<const uint4*>(buf + r32 * kPitch + 16 * (s + half * kSteps / 2) + 8 * h);
#pragma unroll
                for (int s = 0; s < kSteps / 2; ++s)
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, wf[s + half * kSteps / 2]),
                                                                  __builtin_bit_cast(bf16x8, xb[s]), acc, 0, 0, 0);
            }
            float* ob = o_lds[PAR] + r32 * kOPitch + 32 * wave + 4 * h;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                *reinterpret_cast<f32x4*>(ob + 8 * j) = f32x4{acc[4 * j], acc[4 * j + 1], acc[4 * j + 2], acc[4 * j + 3]};
        }
        if (more) store_tile(t + 1, x_lds[PAR ^ 1]);
        __syncthreads();
    };
    for (int64_t t = t_begin; t < t_end; t += 2) {
        iteration(t, std::integral_constant<int, 0>{});
        if (t + 1 < t_end) iteration(t + 1, std::integral_constant<int, 1>{});
    }
}

// The streaming form with its memory traffic on separate waves: waves 0..7
// compute as in linear_stream_kernel, reading x only from LDS and leaving each
// 32 x 256 result tile in one of two LDS buffers; waves 8..11 ("IO waves")
// hold the next two x tiles in registers (loads issued two steps before the
// tile is needed, each instruction one row's 1 KB), round the next step's
// tile to bf16 into LDS, and store the previous step's result tile (one row's
// 1 KB of this column group per instruction). No computing wave waits on
// global memory. Block (row part rp, column group) takes every row_parts-th
// tile from rp, so all blocks write within one moving window of the output
// (361 us against 371 us for consecutive tiles per block). Same products and
// order as linear_stream_kernel (and linear_t32_kernel), same bits. Taken for
// outputs without a residual, 16-byte aligned, N % 4 = 0.
//   262144 x 256 -> 1192: 361 us against 445 us for linear_stream_sw_kernel.
//   Timing copies: the loads and products alone take 220 us, the stores alone
//   310-350 us (a probe writing the same pattern with nothing else takes 335 us,
//   against 230 us for each block writing one contiguous range and 192 us for a
//   fill): the stores bound it. Measured and not kept: a column-blocked output
//   layout ([5][rows][256], each block's stores contiguous: 384-405 us), three or
//   more tiles in flight (the registers spill: 760 us).
template <int I, int U, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < U) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, U>(f);
    }
}

constexpr int kIoWaves = 4;

__global__ __launch_bounds__(64 * (kStreamWaves + kIoWaves))
void linear_stream_io_kernel(LinearArgs p, int col_groups, int row_parts) {
    constexpr int DEPTH = 2;  // x tiles in flight per IO lane (three spill)
    using T = u16;
    constexpr int kSteps = kStreamK / 16;
    constexpr int kPitch = kStreamK + 8;      // x tile row pitch in bf16 (+16 bytes)
    constexpr int kOPitch = kStreamCols + 4;  // output tile row pitch in floats (+16 bytes)
    constexpr int kIoThr = 64 * kIoWaves;
    constexpr int kRowsPerPass = kIoThr / (kStreamK / 4);             // x rows one IO instruction covers (4)
    constexpr int kXLoads = kStreamRows / kRowsPerPass;               // float4 x loads per IO lane per tile (8)
    constexpr int kOStores = kStreamRows * kStreamCols / 4 / kIoThr;  // float4 stores per IO lane per tile (8)
    constexpr int U = 2;                                              // steps per unrolled loop trip
    static_assert(U % DEPTH == 0, "a trip holds whole rotations of the register sets");
    static_assert(kStreamRT == 1 && kStreamK / 4 == 64 && kStreamCols / 4 == 64, "one row per IO instruction");
    __shared__ __attribute__((aligned(16))) T x_lds[2][kStreamRows * kPitch];
    __shared__ __attribute__((aligned(16))) float o_lds[2][kStreamRows * kOPitch];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool io = wave >= kStreamWaves;
    const int xcd = blockIdx.x % 8;
    const int local = blockIdx.x / 8;
    const int cg = local % col_groups;
    const int rpl = local / col_groups;
    const int rp = rpl * 8 + xcd;
    if (rp >= row_parts) return;
    // Step k of the block computes tile rp + k * row_parts.
    const int64_t tiles = (p.rows + kStreamRows - 1) / kStreamRows;
    const int64_t first = rp, tstride = row_parts;
    const int count = static_cast<int>((tiles - rp + row_parts - 1) / row_parts);
    if (count <= 0) return;
    const int64_t n_block = static_cast<int64_t>(cg) * kStreamCols;

    if (io) {
        const int u = 64 * (wave - kStreamWaves) + lane;
        const int ur = u / 64, uc = 4 * (u % 64);  // row within a pass, float column (x and output alike)
        const int64_t col = n_block + uc;
        const bool col_live = col < p.N;
        f32x4 bias4 = {0.f, 0.f, 0.f, 0.f};
        if (p.bias != nullptr && col_live) bias4 = *reinterpret_cast<const f32x4*>(p.bias + col);
        // Nothing in flight before the loop: a load still pending at its head would make the compiler
        // wait for every store of the previous steps where the bias is first used in each step.
        __builtin_amdgcn_s_waitcnt(0);
        // x rows and result rows through buffer resources: a load past the range returns zeros (rows past
        // the end, steps outside the block's) and a store past it is dropped, so no memory operation sits
        // behind a branch and the compiler counts every wave's loads and stores exactly (they share one
        // counter: a store behind a branch made the loads wait for the newest ones). Offsets: a per-lane
        // constant plus a uniform part per step and instruction.
        const int64_t live_cols = p.N - n_block < kStreamCols ? p.N - n_block : kStreamCols;
        const __amdgpu_buffer_rsrc_t x_rsrc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(p.x), 0, static_cast<int>(((p.rows - 1) * p.x_stride + kStreamK) * 4), kBufferWord3);
        const __amdgpu_buffer_rsrc_t out_rsrc = __builtin_amdgcn_make_buffer_rsrc(
            p.out + n_block, 0, static_cast<int>(((p.rows - 1) * p.out_stride + live_cols) * 4), kBufferWord3);
        const uint32_t x_lane = static_cast<uint32_t>((ur * p.x_stride + uc) * 4);
        const uint32_t o_lane = static_cast<uint32_t>((ur * p.out_stride + uc) * 4);
        const uint32_t x_pass = static_cast<uint32_t>(kRowsPerPass * p.x_stride * 4);  // between a lane's rows
        const uint32_t o_pass = static_cast<uint32_t>(kRowsPerPass * p.out_stride * 4);
        constexpr uint32_t kOut = 0x80000000u;  // past every range
        f32x4 xs[DEPTH][kXLoads];
        auto load = [&](auto set_c, int k) __attribute__((always_inline)) {
            constexpr int S = decltype(set_c)::value;
            const int64_t row = (first + k * tstride) * kStreamRows;
            const uint32_t tile = k >= 0 && k < count ? static_cast<uint32_t>(row * p.x_stride * 4) : kOut;
#pragma unroll
            for (int q = 0; q < kXLoads; ++q)
                xs[S][q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, tile + x_lane + q * x_pass, 0, 0));
        };
        auto put = [&](auto set_c, T* buf) __attribute__((always_inline)) {
            constexpr int S = decltype(set_c)::value;
#pragma unroll
            for (int q = 0; q < kXLoads; ++q) {
                const f32x4 v = xs[S][q];
                bf16x4 o;
#pragma unroll
                for (int j = 0; j < 4; ++j) o[j] = static_cast<__bf16>(v[j]);
                *reinterpret_cast<bf16x4*>(buf + (ur + kRowsPerPass * q) * kPitch + uc) = o;
            }
        };
        auto write_out = [&](int k, const float* buf) __attribute__((always_inline)) {
            const int64_t row = (first + k * tstride) * kStreamRows;
            const bool k_live = k >= 0 && k < count;
            const uint32_t tile = static_cast<uint32_t>(row * p.out_stride * 4);
            const int64_t rows_left = p.rows - row;  // rows of this tile that exist
#pragma unroll
            for (int i = 0; i < kOStores; ++i) {
                const int rr = ur + kRowsPerPass * i;
                f32x4 y = *reinterpret_cast<const f32x4*>(buf + rr * kOPitch + uc);
                if (p.bias != nullptr) y += bias4;
                const bool live = k_live & col_live & (rr < rows_left);
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, y), out_rsrc, live ? tile + o_lane + i * o_pass : kOut, 0, 0);
            }
        };
        // Step k's x tile lives in register set k % DEPTH. The loop starts DEPTH + 1 steps early (loads
        // before the block's steps read past the range, stores before them are dropped, the LDS tiles
        // they write are never read): the first real step then sees the same operations in flight as
        // every later one, and the compiler's count at the loop head is the steady state's.
        auto io_step = [&](auto i_c, int k) __attribute__((always_inline)) {
            constexpr int I = decltype(i_c)::value;  // k + DEPTH + 1 = I (mod U)
            constexpr int S = I % DEPTH;             // the set of step k + 1
            constexpr int B = (I + DEPTH) & 1;       // the LDS buffers of steps k + 1 and k - 1
            if (k + 1 < count) put(std::integral_constant<int, S>{}, x_lds[B]);
            __builtin_amdgcn_sched_barrier(0);  // the set is free only after its LDS writes
            load(std::integral_constant<int, S>{}, k + 1 + DEPTH);
            __builtin_amdgcn_sched_barrier(0);
            write_out(k - 1, o_lds[B]);
            __syncthreads();
        };
        // Whole trips of U steps without a branch around their memory operations, then the rest.
        int k0 = -DEPTH - 1;
        for (; k0 + U <= count; k0 += U) static_for<0, U>([&](auto i_c) { io_step(i_c, k0 + decltype(i_c)::value); });
        static_for<0, U>([&](auto i_c) {
            if (k0 + decltype(i_c)::value < count) io_step(i_c, k0 + decltype(i_c)::value);
        });
        write_out(count - 1, o_lds[(count - 1) & 1]);
        return;
    }

    const int r32 = lane & 31;
    const int h = lane >> 5;
    const int64_t n_wave = n_block + 32 * wave;
    const bool wave_live = n_wave < p.N;
    uint4 wf[kSteps];
    {
        const T* w = static_cast<const T*>(p.w);
        const int64_t n = n_wave + r32;
        const T* wrow = w + (n < p.N ? n : p.N - 1) * kStreamK + 8 * h;
        const uint32_t keep = n < p.N ? 0xffffffffu : 0u;
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const uint4 v = *reinterpret_cast<const uint4*>(wrow + 16 * s);
            wf[s] = uint4{v.x & keep, v.y & keep, v.z & keep, v.w & keep};
        }
    }
    for (int k = 0; k <= DEPTH; ++k) __syncthreads();  // the IO waves' steps before the block's
    auto step = [&](auto par_c) __attribute__((always_inline)) {
        constexpr int PAR = decltype(par_c)::value;  // k % 2: the buffers of step k
        if (wave_live) {
            const T* buf = x_lds[PAR];
            f32x16 acc;
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
            uint4 xb[kSteps];
#pragma unroll
            for (int s = 0; s < kSteps; ++s) xb[s] = *reinterpret_cast<const uint4*>(buf + r32 * kPitch + 16 * s + 8 * h);
#pragma unroll
            for (int s = 0; s < kSteps; ++s)
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, wf[s]),
                                                              __builtin_bit_cast(bf16x8, xb[s]), acc, 0, 0, 0);
            float* ob = o_lds[PAR] + r32 * kOPitch + 32 * wave + 4 * h;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                *reinterpret_cast<f32x4*>(ob + 8 * j) = f32x4{acc[4 * j], acc[4 * j + 1], acc[4 * j + 2], acc[4 * j + 3]};
        }
        __syncthreads();
    };
    for (int k = 0; k < count; k += 2) {
        step(std::integral_constant<int, 0>{});
        if (k + 1 < count) step(std::integral_constant<int, 1>{});
    }
}

// Shapes too small to give the 128-row blocks one per CU (256 CUs), with K
// held in at most eight 32-wide steps.
// linear_tiles_kernel's BUF form: K a multiple of the 16-byte unit (kper elements), N % 4 = 0, 16-byte
// aligned output (and residual) rows, the output within 2 GiB.
bool tiles_buf_fits(const LinearArgs& p, int64_t rows, int kper) {
    auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    return p.K % kper == 0 && p.N % 4 == 0 && a16(p.out) && p.out_stride % 4 == 0 &&
           (p.residual == nullptr || (a16(p.residual) && p.res_stride % 4 == 0)) &&
           (rows + 1) * p.out_stride * 4 < (int64_t{1} << 31);
}

bool small_shape(int64_t rows, int64_t K, int64_t N) {
    return K % 8 == 0 && K <= 256 && ceil_div(rows, kRowsPerBlock) * ceil_div(N, kColsPerChunk) < 256 &&
           ceil_div(rows, 16) * ceil_div(N, 16) <= 0x7fffffff;
}

// MLK_LINEAR_FORM=t32 keeps linear_t32_kernel for the shapes the streaming form takes (read at each
// call, so a caller can compare the two forms).
bool stream_form() {
    const char* v = std::getenv("MLK_LINEAR_FORM");
    return !(v != nullptr && std::strcmp(v, "t32") == 0);
}

// MLK_LINEAR_STORE_WAVES selects the streaming form: unset (or "io") the IO-wave form where the output
// allows it, "sw" the form with storing waves only, "0" the one without either.
int store_waves() {
    const char* v = std::getenv("MLK_LINEAR_STORE_WAVES");
    if (v != nullptr && std::strcmp(v, "0") == 0) return 0;
    if (v != nullptr && std::strcmp(v, "sw") == 0) return 1;
    return 2;
}

// The IO-wave form: no residual, 16-byte aligned output rows and bias, N % 4 = 0, and x and the output
// within the 2 GiB a buffer offset reaches.
// linear_stream_kernel's buffer-store epilogue: no bias or residual, N % 4 = 0, 16-byte aligned output
// rows within 2 GiB.
bool buf_out_fits(const LinearArgs& p, int64_t rows) {
    return p.residual == nullptr && p.bias == nullptr && p.N % 4 == 0 && (reinterpret_cast<uintptr_t>(p.out) & 15) == 0 &&
           p.out_stride % 4 == 0 && (rows + 1) * p.out_stride * 4 < (int64_t{1} << 31);
}

bool io_form_fits(const LinearArgs& p, int64_t rows) {
    auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    const int64_t span = (rows + kStreamRows) * (p.out_stride > p.x_stride ? p.out_stride : p.x_stride) * 4;
    return p.residual == nullptr && p.N % 4 == 0 && a16(p.out) && p.out_stride % 4 == 0 &&
           (p.bias == nullptr || a16(p.bias)) && span < (int64_t{1} << 31);
}

template <bool BF16W, bool VEC>
void launch(const LinearArgs& p, int64_t rows, int64_t n_chunks, hipStream_t stream) {
    constexpr int KC = WTraits<BF16W>::kKChunk;
    // Shapes too small to give the 128-row blocks one per CU (256 CUs) take
    // one wave per 16 x 16 tile (2048 x 128 -> 64: 16 blocks of the tiled
    // form, 512 waves here).
    const int64_t tiles = ceil_div(rows, 16) * ceil_div(p.N, 16);
    if (VEC && small_shape(rows, p.K, p.N)) {
        if (p.K <= 64) {
            launch_small<BF16W, 2>(p, tiles, stream);
        } else if (p.K <= 128) {
            launch_small<BF16W, 4>(p, tiles, stream);
        } else {
            launch_small<BF16W, 8>(p, tiles, stream);
        }
        return;
    }
    // bf16 weights with K within one chunk and a wide output (12 or more
    // 64-column chunks): the 32 x 32 x 16 form, 256 rows per block (262144 x
    // 256 -> 1192: 577 -> 513 us). Narrower outputs keep the 16 x 16 x 32
    // form, whose smaller blocks give more parallelism (32768 x 256 -> 336:
    // 28 us against 42 us; 262144 x 40 -> 256: 90 against 129 us).
    if constexpr (BF16W) {
        if (VEC && p.K == kStreamK && p.x_stride % 4 == 0 && n_chunks >= 12 && stream_form()) {
            const int col_groups = static_cast<int>(ceil_div(p.N, kStreamCols));
            // One block per CU (256 CUs): per XCD 32 block slots, whole row parts of col_groups blocks each.
            const int parts_per_xcd = 32 / col_groups;
            if (parts_per_xcd >= 1) {
                const int row_parts = 8 * parts_per_xcd;
                const dim3 grid(static_cast<unsigned>(8 * parts_per_xcd * col_groups));
                const int form = store_waves();
                if (form == 2 && io_form_fits(p, rows)) {
                    hipLaunchKernelGGL(linear_stream_io_kernel, grid, dim3(64 * (kStreamWaves + kIoWaves)), 0, stream, p,
                                       col_groups, row_parts);
                } else if (form >= 1) {
                    hipLaunchKernelGGL(linear_stream_sw_kernel, grid, dim3(64 * (kStreamWaves + kStoreWaves)), 0,
                                       stream, p, col_groups, row_parts);
                } else {
                    hipLaunchKernelGGL(linear_stream_kernel<kStreamK>, grid, dim3(64 * kStreamWaves), 0, stream, p,
                                       col_groups, row_parts);
                }
                return;
            }
        }
        // K = 512 (the stack's Mamba out_proj, 262144 x 512 -> 256): the streaming form with 128 registers of
        // W fragments per wave, two waves per SIMD (no storing waves: they would leave 168 registers);
        // 288 -> 190 us against the tiled 16 x 16 x 32 form.
        if (VEC && p.K == 512 && p.x_stride % 4 == 0 && p.N >= 128 && rows >= 32768 && stream_form()) {
            const int col_groups = static_cast<int>(ceil_div(p.N, kStreamCols));
            const int parts_per_xcd = 32 / col_groups;
            if (parts_per_xcd >= 1) {
                const int row_parts = 8 * parts_per_xcd;
                const dim3 grid(static_cast<unsigned>(8 * parts_per_xcd * col_groups));
                if (buf_out_fits(p, rows)) {
                    hipLaunchKernelGGL((linear_stream_kernel<512, true>), grid, dim3(64 * kStreamWaves), 0, stream, p,
                                       col_groups, row_parts);
                } else {
                    hipLaunchKernelGGL((linear_stream_kernel<512, false>), grid, dim3(64 * kStreamWaves), 0, stream, p,
                                       col_groups, row_parts);
                }
                return;
            }
        }
        if (p.K <= KC && n_chunks >= 12) {
            const int64_t row_blocks32 = ceil_div(rows, 2 * kRowsPerBlock);
            int64_t gy32 = 1;
            while (gy32 < n_chunks && row_blocks32 * gy32 < 512) ++gy32;
            hipLaunchKernelGGL((linear_t32_kernel<VEC>), dim3(static_cast<unsigned>(row_blocks32), static_cast<unsigned>(gy32)),
                               dim3(kThreads), 0, stream, p);
            return;
        }
    }
    // gy splits N only while there are fewer than ~512 blocks (two per CU).
    // Two row tiles per wave (half the LDS reads of W per row) measured
    // slower at 262144 x 256 -> 1192 (0.64 vs 0.58 ms): the register budget
    // leaves one block per CU.
    const int64_t row_blocks = ceil_div(rows, kRowsPerBlock);
    int64_t gy = 1;
    while (gy < n_chunks && row_blocks * gy < 512) ++gy;
    const dim3 grid(static_cast<unsigned>(row_blocks), static_cast<unsigned>(gy));
    // fp32 weights within one K chunk keep the row-layout kernel (measured
    // faster there: 7.2 vs 8.6 us at 2048 x 64 -> 304, 71 vs 79 us at
    // 65536 x 128 -> 257); bf16 weights take the tiled kernel (27.6 vs 29.3 us
    // at 32768 x 256 -> 336).
    if (p.K <= KC && !BF16W) {
        hipLaunchKernelGGL((linear_kernel<BF16W, VEC, false>), grid, dim3(kThreads), 0, stream, p);
    } else if (p.K <= KC) {
        // (KS = 1 keeps four waves per SIMD: the residual's registers would spill, so it takes BUF = 1 only)
        if (VEC && p.residual == nullptr && tiles_buf_fits(p, rows, 16 / static_cast<int>(sizeof(typename WTraits<BF16W>::T)))) {
            hipLaunchKernelGGL((linear_tiles_kernel<BF16W, VEC, 1, 1, VEC ? 1 : 0>), grid, dim3(kThreads), 0, stream, p);
        } else {
            hipLaunchKernelGGL((linear_tiles_kernel<BF16W, VEC, 1, 1>), grid, dim3(kThreads), 0, stream, p);
        }
    } else if (p.K <= 2 * KC) {
        if (VEC && p.residual == nullptr && tiles_buf_fits(p, rows, 16 / static_cast<int>(sizeof(typename WTraits<BF16W>::T)))) {
            hipLaunchKernelGGL((linear_tiles_kernel<BF16W, VEC, 1, 2, VEC ? 1 : 0>), grid, dim3(kThreads), 0, stream, p);
        } else if (VEC && tiles_buf_fits(p, rows, 16 / static_cast<int>(sizeof(typename WTraits<BF16W>::T)))) {
            hipLaunchKernelGGL((linear_tiles_kernel<BF16W, VEC, 1, 2, VEC ? 2 : 0>), grid, dim3(kThreads), 0, stream, p);
        } else {
            hipLaunchKernelGGL((linear_tiles_kernel<BF16W, VEC, 1, 2>), grid, dim3(kThreads), 0, stream, p);
        }
    } else {
        hipLaunchKernelGGL((linear_kernel<BF16W, VEC, true>), grid, dim3(kThreads), 0, stream, p);
    }
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
    const int64_t n_chunks = ceil_div(out_features, kColsPerChunk);
    MLK_CHECK(ceil_div(rows, kRowsPerBlock) <= 0x7fffffff, "too many rows");
    const size_t wsize = weight_dtype == MLK_DTYPE_BF16 ? 2 : 4;
    const bool vec = aligned16(x) && x_stride % 4 == 0 && aligned16(weight) && (in_features * wsize) % 16 == 0;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (weight_dtype == MLK_DTYPE_BF16) {
        vec ? launch<true, true>(p, rows, n_chunks, s) : launch<true, false>(p, rows, n_chunks, s);
    } else {
        vec ? launch<false, true>(p, rows, n_chunks, s) : launch<false, false>(p, rows, n_chunks, s);
    }
    return launch_status("linear");
}

extern "C" mlk_status mlk_linear_residual(const float* x, int64_t rows, int64_t in_features, int64_t x_stride,
                                          const void* weight, int32_t weight_dtype, const float* bias,
                                          int64_t out_features, const float* residual, int64_t res_stride,
                                          float* out, int64_t out_stride, mlk_stream_t stream) {
    MLK_CHECK(rows >= 0 && in_features > 0 && out_features > 0, "invalid linear geometry");
    MLK_CHECK(x_stride >= in_features, "x row stride must be at least in_features");
    MLK_CHECK(out_stride >= out_features, "out row stride must be at least out_features");
    MLK_CHECK(res_stride >= out_features, "residual row stride must be at least out_features");
    MLK_CHECK(weight_dtype == MLK_DTYPE_F32 || weight_dtype == MLK_DTYPE_BF16, "weight dtype must be f32 or bf16");
    if (rows == 0) return MLK_OK;
    MLK_CHECK(x && weight && out && residual, "null tensor pointer");
    MLK_CHECK(ceil_div(rows, kRowsPerBlock) <= 0x7fffffff, "too many rows");
    LinearArgs p{x, rows, in_features, x_stride, weight, bias, out_features, out, out_stride, residual, res_stride};
    const int64_t n_chunks = ceil_div(out_features, kColsPerChunk);
    const size_t wsize = weight_dtype == MLK_DTYPE_BF16 ? 2 : 4;
    const bool vec = aligned16(x) && x_stride % 4 == 0 && aligned16(weight) && (in_features * wsize) % 16 == 0;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (weight_dtype == MLK_DTYPE_BF16) {
        vec ? launch<true, true>(p, rows, n_chunks, s) : launch<true, false>(p, rows, n_chunks, s);
    } else {
        vec ? launch<false, true>(p, rows, n_chunks, s) : launch<false, false>(p, rows, n_chunks, s);
    }
    return launch_status("linear_residual");
}

extern "C" mlk_status mlk_rms_norm_linear(const float* x, int64_t rows, int64_t in_features, int64_t x_stride,
                                          const float* norm_weight, double eps, int64_t groups, const void* weight,
                                          int32_t weight_dtype, const float* bias, int64_t out_features, float* out,
                                          int64_t out_stride, mlk_stream_t stream) {
    MLK_CHECK(rows >= 0 && in_features > 0 && out_features > 0, "invalid linear geometry");
    MLK_CHECK(groups > 0 && in_features % groups == 0, "groups must divide the normalised dimension");
    MLK_CHECK(x_stride >= in_features, "x row stride must be at least in_features");
    MLK_CHECK(out_stride >= out_features, "out row stride must be at least out_features");
    MLK_CHECK(weight_dtype == MLK_DTYPE_F32 || weight_dtype == MLK_DTYPE_BF16, "weight dtype must be f32 or bf16");
    const int64_t gs = in_features / groups;
    const size_t wsize = weight_dtype == MLK_DTYPE_BF16 ? 2 : 4;
    const bool vec = aligned16(x) && x_stride % 4 == 0 && aligned16(weight) && (in_features * wsize) % 16 == 0 &&
                     aligned16(norm_weight);
    const bool gs_ok = gs == 8 || gs == 16 || gs == 32 || gs == 64;
    // Large row counts: the row-layout kernel with the prologue, for fp32 weights and K of one chunk.
    const bool rows_form = vec && gs_ok && !small_shape(rows, in_features, out_features) &&
                           weight_dtype == MLK_DTYPE_F32 && in_features == WTraits<false>::kKChunk;
    if (!vec || !gs_ok || !(small_shape(rows, in_features, out_features) || rows_form)) {
        set_error("rms_norm_linear: shape without the fused form (use rms_norm then linear)");
        return MLK_ERR_UNSUPPORTED;
    }
    if (rows == 0) return MLK_OK;
    MLK_CHECK(x && norm_weight && weight && out, "null tensor pointer");
    LinearArgs p{x, rows, in_features, x_stride, weight, bias, out_features, out, out_stride, nullptr, 0,
                 norm_weight, static_cast<double>(static_cast<float>(eps))};
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (rows_form) {
        MLK_CHECK(ceil_div(rows, kRowsPerBlock) <= 0x7fffffff, "too many rows");
        const int64_t n_chunks = ceil_div(out_features, kColsPerChunk);
        const int64_t row_blocks = ceil_div(rows, kRowsPerBlock);
        int64_t gy = 1;
        while (gy < n_chunks && row_blocks * gy < 512) ++gy;
        const dim3 grid(static_cast<unsigned>(row_blocks), static_cast<unsigned>(gy));
        const bool buf = (rows + 1) * out_stride * 4 < (int64_t{1} << 31);
#define MLK_ROWS_GS(G)                                                                                              \
    do {                                                                                                            \
        if (buf) {                                                                                                  \
            hipLaunchKernelGGL((linear_kernel<false, true, false, G, true>), grid, dim3(kThreads), 0, s, p);        \
        } else {                                                                                                    \
            hipLaunchKernelGGL((linear_kernel<false, true, false, G>), grid, dim3(kThreads), 0, s, p);              \
        }                                                                                                           \
    } while (0)
        switch (gs) {
            case 8: MLK_ROWS_GS(8); break;
            case 16: MLK_ROWS_GS(16); break;
            case 32: MLK_ROWS_GS(32); break;
            default: MLK_ROWS_GS(64); break;
        }
#undef MLK_ROWS_GS
        return launch_status("rms_norm_linear");
    }
    const int64_t tiles = ceil_div(rows, 16) * ceil_div(out_features, 16);
#define MLK_NORM_GS(G)                                                                             \
    (weight_dtype == MLK_DTYPE_BF16 ? launch_small_norm<true, G>(p, tiles, s) : launch_small_norm<false, G>(p, tiles, s))
    switch (gs) {
        case 8: MLK_NORM_GS(8); break;
        case 16: MLK_NORM_GS(16); break;
        case 32: MLK_NORM_GS(32); break;
        default: MLK_NORM_GS(64); break;
    }
#undef MLK_NORM_GS
    return launch_status("rms_norm_linear");
}
