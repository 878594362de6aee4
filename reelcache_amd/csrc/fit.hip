// Fit-side kernels for MI355X (gfx950): max|X|, batched symmetric Gram, projection onto a
// stored fp16 basis, direct residual / source energies, column extrema and the 8-bit quantizer.
//
// Reference: reelcache/gpu_fitting.py (gram_bases :276-295), reelcache/rank_method.py
// (_symmetric_gram :634-638), reelcache/factorization.py (project_onto_basis :318-434,
// measure_source_energy :692-724), reelcache/node_packets.py (quantize_device :155-173),
// reelcache/_hevc.py (quantize_coefficients :445-472).
//
// Arithmetic contract:
//   * Gram: exact products (16-bit sources on 16-bit MFMA, whose products are exact in fp32;
//     fp32 sources on fp32 MFMA), fp32 accumulation, exactly symmetric output.
//   * Projection P = X Q^T and the reconstruction P Q of the residual: operands converted
//     exactly to FP64, products and sums on v_mfma_f64_16x16x4f64, P rounded once to fp32.
//     The FP64 sum makes P the correctly rounded fp32 value of the exact dot product except
//     within ~1e-13 relative of a rounding boundary, i.e. independent of summation order.
//   * Energies: FP64 sums of (x - r)^2 and x^2, divided by s^2 per 64-row partial, fixed-order totals.
//   * Quantizer: FP64 (v - offset) / scale, round half to even, clamp to [0, 255].
#include <type_traits>

#include "common.h"

namespace rch {
namespace {

constexpr int kThreads = 256;

template <int DT>
constexpr int esize() {
    return DT == RCH_DT_F32 ? 4 : 2;
}

// 16-bit element bits -> float.
template <int DT>
__device__ __forceinline__ float half_bits(uint32_t bits) {
    if constexpr (DT == RCH_DT_BF16) {
        return __uint_as_float(bits << 16);
    } else {
        return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
    }
}

// Eight consecutive source elements as doubles.
template <int DT>
__device__ __forceinline__ void load8(__amdgpu_buffer_rsrc_t rsrc, uint32_t offset, double (&v)[8]) {
    if constexpr (DT == RCH_DT_F32) {
        const u4 a = __builtin_amdgcn_raw_buffer_load_b128(rsrc, offset, 0, 0);
        const u4 b = __builtin_amdgcn_raw_buffer_load_b128(rsrc, offset + 16, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = static_cast<double>(__uint_as_float(a[i]));
            v[4 + i] = static_cast<double>(__uint_as_float(b[i]));
        }
    } else {
        const u4 w = __builtin_amdgcn_raw_buffer_load_b128(rsrc, offset, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = static_cast<double>(half_bits<DT>(w[i] & 0xffffu));
            v[2 * i + 1] = static_cast<double>(half_bits<DT>(w[i] >> 16));
        }
    }
}

// Order-preserving unsigned key of an fp32 value (larger value -> larger key).
__device__ __forceinline__ uint32_t order_key(float v) {
    const uint32_t u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Buffer over rows [r0, rows) of a source matrix (empty when r0 >= rows).
template <int DT>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t source_rows(const rch_fit_matrix* M, int channels, int64_t r0) {
    constexpr int E = esize<DT>();
    const int64_t left = M->rows - r0;
    return make_rsrc(M->src_ptr + r0 * M->src_stride * E, left > 0 ? ((left - 1) * M->src_stride + channels) * E : 0);
}

// ---------------------------------------------------------------------------------------------
// max|X|: workgroup (64-row tile, matrix); one unsigned atomic max of the fp32 bits per workgroup.
// ---------------------------------------------------------------------------------------------

template <int DT>
__global__ void __launch_bounds__(kThreads) absmax_kernel(const rch_fit_matrix* __restrict__ mats, int channels) {
    const rch_fit_matrix* M = mats + blockIdx.y;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * 64;
    if (r0 >= M->rows) return;
    constexpr int E = esize<DT>();
    const int rows = static_cast<int>(M->rows - r0 < 64 ? M->rows - r0 : 64);
    const __amdgpu_buffer_rsrc_t src = source_rows<DT>(M, channels, r0);
    const int groups = channels / 8;  // 8 elements per load
    uint32_t m = 0;
    for (int i = threadIdx.x; i < rows * groups; i += kThreads) {
        const int r = i / groups, g = i - r * groups;
        double v[8];
        load8<DT>(src, static_cast<uint32_t>((r * M->src_stride + 8 * g) * E), v);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t bits = __float_as_uint(static_cast<float>(v[j])) & 0x7fffffffu;  // exact: v is a float
            m = bits > m ? bits : m;
        }
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        const uint32_t o = __shfl_xor(m, d);
        m = o > m ? o : m;
    }
    __shared__ uint32_t part[kThreads / 64];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kThreads / 64; ++w) m = part[w] > m ? part[w] : m;
        atomicMax(reinterpret_cast<unsigned int*>(M->absmax_ptr), m);  // vector atomic
    }
}

// ---------------------------------------------------------------------------------------------
// Gram G = X^T X.  Workgroup = one 256 x 256 tile (ti >= tj) of one matrix, 16 waves: wave w
// computes the 64 x 64 quadrant (w / 4, w % 4) as 2 x 2 MFMA 32x32 blocks (on a diagonal tile
// the quadrants above the diagonal are mirrors and are skipped), and stages a quarter of the
// step's rows for 128 channels of one panel.  Rows are staged 32 per step into LDS as
// [channel][row]: each lane loads a channel pair of 8 rows, coalesced along the row, and writes
// the two channels' row runs, so that an MFMA operand (8 consecutive rows of one channel for
// 16-bit sources, 16 for fp32) is one or four 16-byte LDS reads.  Register-prefetched two steps
// ahead, double-buffered LDS, one barrier per step.
//
// The 21 tiles of a 1536-channel matrix run on one XCD (xcd_unit) and sweep the rows together,
// so each row band of X is fetched from HBM about once and then read from that XCD's L2 by the
// six tiles of each panel.  Every output element sums its products in row order, 16 rows (2 for
// fp32) per MFMA, so the result does not depend on the tile size or the rows per step.
// ---------------------------------------------------------------------------------------------

constexpr int kGramTile = 256;
constexpr int kGramThreads = 1024;

// Rows staged per step (a wave stages a quarter of them).  Measured on MI355X, 32-row steps with
// loads two steps ahead beat 64-row steps (which leave registers for one step ahead only).
template <int DT>
constexpr int gram_rows() {
    return 32;
}

template <int DT>
constexpr int gram_pitch() {
    return gram_rows<DT>() * esize<DT>() + 16;  // bytes per staged channel
}

template <int DT>
struct GramStage {
    typedef typename std::conditional<DT == RCH_DT_F32, u2, uint32_t>::type word;
    word d[gram_rows<DT>() / 4];  // rows r0 .. of this lane's channel pair
};

template <int DT>
__device__ __forceinline__ void gram_load(GramStage<DT>& st, const rch_fit_matrix* M, int channels, int64_t r0, int c) {
    constexpr int E = esize<DT>();
    const __amdgpu_buffer_rsrc_t src = source_rows<DT>(M, channels, r0);
    const uint32_t offset = c < channels ? static_cast<uint32_t>(c * E) : kOutOfRange;
    const uint32_t row_bytes = static_cast<uint32_t>(M->src_stride * E);
#pragma unroll
    for (int r = 0; r < gram_rows<DT>() / 4; ++r) {
        if constexpr (DT == RCH_DT_F32)
            st.d[r] = __builtin_amdgcn_raw_buffer_load_b64(src, offset + r * row_bytes, 0, 0);
        else
            st.d[r] = __builtin_amdgcn_raw_buffer_load_b32(src, offset + r * row_bytes, 0, 0);
    }
}

// The stage's two channels, each as a run of rows/4 consecutive rows at row offset
// group * rows / 4 of the channel's staged row block.
template <int DT>
__device__ __forceinline__ void gram_store(const GramStage<DT>& st, unsigned char* tile, int lane, int group) {
    constexpr int P = gram_pitch<DT>();
    unsigned char* c0 = tile + (2 * lane) * P;
    unsigned char* c1 = c0 + P;
    if constexpr (DT == RCH_DT_F32) {
        static_assert(gram_rows<DT>() == 32, "fp32 stages hold 8 rows per lane");
        const u4 a0 = {st.d[0][0], st.d[1][0], st.d[2][0], st.d[3][0]};
        const u4 a1 = {st.d[4][0], st.d[5][0], st.d[6][0], st.d[7][0]};
        const u4 b0 = {st.d[0][1], st.d[1][1], st.d[2][1], st.d[3][1]};
        const u4 b1 = {st.d[4][1], st.d[5][1], st.d[6][1], st.d[7][1]};
        *reinterpret_cast<u4*>(c0 + 32 * group) = a0;
        *reinterpret_cast<u4*>(c0 + 32 * group + 16) = a1;
        *reinterpret_cast<u4*>(c1 + 32 * group) = b0;
        *reinterpret_cast<u4*>(c1 + 32 * group + 16) = b1;
    } else {
        constexpr int kRuns = gram_rows<DT>() / 32;  // 8-row runs (16 bytes) per lane and channel
        static_assert(kRuns >= 1 && 8 * kRuns == sizeof(st.d) / sizeof(st.d[0]), "stage rows");
#pragma unroll
        for (int run = 0; run < kRuns; ++run) {  // rows 8 run .. 8 run + 7 of the stage
            u4 lo, hi;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t even = st.d[8 * run + 2 * q], odd = st.d[8 * run + 2 * q + 1];
                lo[q] = (even & 0xffffu) | (odd << 16);
                hi[q] = (even >> 16) | (odd & 0xffff0000u);
            }
            *reinterpret_cast<u4*>(c0 + 16 * kRuns * group + 16 * run) = lo;
            *reinterpret_cast<u4*>(c1 + 16 * kRuns * group + 16 * run) = hi;
        }
    }
}

template <int DT>
__device__ __forceinline__ void gram_mfma(f16v (&acc)[2][2], const unsigned char* ti, const unsigned char* tj, int wm,
                                          int wn, int lane) {
    constexpr int P = gram_pitch<DT>();
    const int h = lane >> 5, col = lane & 31;
    const unsigned char* a_base = ti + (wm * 64 + col) * P;
    const unsigned char* b_base = tj + (wn * 64 + col) * P;
    if constexpr (DT == RCH_DT_F32) {
        // Lane half h holds rows 16h .. 16h + 15; MFMA step s takes row 16h + s.
        f4 a[2][4], b[2][4];
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                a[x][q] = *reinterpret_cast<const f4*>(a_base + x * 32 * P + 64 * h + 16 * q);
                b[x][q] = *reinterpret_cast<const f4*>(b_base + x * 32 * P + 64 * h + 16 * q);
            }
#pragma unroll
        for (int s = 0; s < 16; ++s)
#pragma unroll
            for (int x = 0; x < 2; ++x)
#pragma unroll
                for (int y = 0; y < 2; ++y)
                    acc[x][y] =
                        __builtin_amdgcn_mfma_f32_32x32x2f32(a[x][s >> 2][s & 3], b[y][s >> 2][s & 3], acc[x][y], 0, 0, 0);
    } else {
        // 16-row MFMA steps; lane half h holds rows 16 ks + 8h .. + 7.
#pragma unroll
        for (int ks = 0; ks < gram_rows<DT>() / 16; ++ks) {
            u4 a[2], b[2];
#pragma unroll
            for (int x = 0; x < 2; ++x) {
                a[x] = *reinterpret_cast<const u4*>(a_base + x * 32 * P + 32 * ks + 16 * h);
                b[x] = *reinterpret_cast<const u4*>(b_base + x * 32 * P + 32 * ks + 16 * h);
            }
#pragma unroll
            for (int x = 0; x < 2; ++x)
#pragma unroll
                for (int y = 0; y < 2; ++y) {
                    if constexpr (DT == RCH_DT_BF16)
                        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf8, a[x]),
                                                                            __builtin_bit_cast(bf8, b[y]), acc[x][y], 0, 0, 0);
                    else
                        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8, a[x]),
                                                                           __builtin_bit_cast(h8, b[y]), acc[x][y], 0, 0, 0);
                }
        }
    }
}

template <int DT>
__global__ void __launch_bounds__(kGramThreads) gram_kernel(const rch_fit_matrix* __restrict__ mats, int channels,
                                                            int tiles, int grid) {
    constexpr int P = gram_pitch<DT>();
    __shared__ __attribute__((aligned(16))) unsigned char lds[2][2][kGramTile * P];

    const int unit = xcd_unit(blockIdx.x, grid);  // the tiles of one matrix share an XCD's L2
    const int mat = unit / tiles;
    int ti = 0, rest = unit - mat * tiles;
    while (rest > ti) {  // tile index -> (ti, tj), row-major over the lower triangle
        rest -= ti + 1;
        ++ti;
    }
    const int tj = rest;
    const bool diagonal = ti == tj;
    const rch_fit_matrix* M = mats + mat;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    // Staging role: panel (0: the ti columns, 1: the tj columns), 128-channel half, 8-row group.
    const int panel = wave >> 3, half = (wave >> 2) & 1, group = wave & 3;
    // A diagonal tile stages one panel: the other panel's waves load from an out-of-range column
    // (the buffer loads return zeros without a memory access), so every wave runs the same
    // straight-line loop and the loads stay in flight across the MFMAs.
    const int c = diagonal && panel == 1 ? channels : (panel ? tj : ti) * kGramTile + 128 * half + 2 * lane;
    // MFMA role: the 64 x 64 quadrant (wm, wn).
    const int wm = wave >> 2, wn = wave & 3;
    const bool computes = !(diagonal && wm < wn);
    constexpr int kRows = gram_rows<DT>();
    const int steps = static_cast<int>((M->rows + kRows - 1) / kRows);

    f16v acc[2][2];
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y) acc[x][y] = f16v{};

    // 16-bit rows are loaded two steps ahead into alternating register stages: the loads for
    // step s + 2 are issued before step s's MFMAs and written to LDS after step s + 1's, so two
    // steps of MFMA work cover their latency.  Rows past the end read as zeros (empty buffer), so
    // the loads and stores need no conditions and the loop stays straight-line, which keeps the
    // compiler's waits on the older stage only.
    unsigned char* staged = lds[0][panel] + 128 * half * P;  // this wave's rows in buffer 0
    constexpr int kBuffer = 2 * kGramTile * P;                // buffer 1 = buffer 0 + kBuffer
    auto mfma_step = [&](int step) {
        const int buf = step & 1;
        if (computes) gram_mfma<DT>(acc, lds[buf][0], diagonal ? lds[buf][0] : lds[buf][1], wm, wn, lane);
        return staged + (buf ^ 1) * kBuffer;  // where the next step's rows go
    };
    if constexpr (DT != RCH_DT_F32) {
        GramStage<DT> sa, sb;
        gram_load<DT>(sa, M, channels, kRows / 4 * group, c);
        gram_load<DT>(sb, M, channels, kRows + kRows / 4 * group, c);
        gram_store<DT>(sa, staged, lane, group);
        __syncthreads();
        auto step_body = [&](int step, GramStage<DT>& ahead, const GramStage<DT>& next) {
            gram_load<DT>(ahead, M, channels, static_cast<int64_t>(step + 2) * kRows + kRows / 4 * group, c);
            gram_store<DT>(next, mfma_step(step), lane, group);
            __syncthreads();
        };
        for (int step = 0; step < steps; step += 2) {
            step_body(step, sa, sb);
            if (step + 1 < steps) step_body(step + 1, sb, sa);
        }
    } else {  // fp32 stages are twice as large: one step ahead keeps the loop within 128 VGPRs
        GramStage<DT> st;
        gram_load<DT>(st, M, channels, kRows / 4 * group, c);
        gram_store<DT>(st, staged, lane, group);
        __syncthreads();
        for (int step = 0; step < steps; ++step) {
            gram_load<DT>(st, M, channels, static_cast<int64_t>(step + 1) * kRows + kRows / 4 * group, c);
            gram_store<DT>(st, mfma_step(step), lane, group);
            __syncthreads();
        }
    }
    if (!computes) return;

    // Accumulator element e of lane l: row 8 (e / 4) + 4 (l / 32) + e % 4, column l % 32.
    RCH_GLOBAL float* G = gout<float>(M->gram_ptr);
    const int64_t ld = M->gram_stride;
    const int h = lane >> 5, col = lane & 31;
    const bool lower_only = diagonal && wm == wn;  // a quadrant on the diagonal: its lower half, mirrored
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y) {
            const int ib = ti * kGramTile + wm * 64 + x * 32;
            const int64_t j = tj * kGramTile + wn * 64 + y * 32 + col;
            if (j >= channels) continue;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int64_t i0 = ib + 8 * g + 4 * h;  // rows i0 .. i0 + 3 (channels % 8 == 0: all or none in range)
                if (i0 >= channels) continue;
                if (!lower_only) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) G[(i0 + r) * ld + j] = acc[x][y][4 * g + r];
                    // Mirror: G[j][i0 .. i0 + 3] is one 16-byte store.
                    const f4 v = {acc[x][y][4 * g], acc[x][y][4 * g + 1], acc[x][y][4 * g + 2], acc[x][y][4 * g + 3]};
                    *reinterpret_cast<RCH_GLOBAL f4*>(G + j * ld + i0) = v;
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int64_t i = i0 + r;
                        if (i >= j) {  // lower triangle, mirrored
                            G[i * ld + j] = acc[x][y][4 * g + r];
                            G[j * ld + i] = acc[x][y][4 * g + r];
                        }
                    }
                }
            }
        }
}

// ---------------------------------------------------------------------------------------------
// Projection P = X Q^T on v_mfma_f64_16x16x4f64: D[m = token][n = rank] = sum_c X[token][c] Q[rank][c].
// Workgroup (64-token tile, 64-rank chunk, matrix); wave w owns tokens 16w .. 16w + 15 of the
// tile and the chunk's 4 rank blocks of 16.  Per 32-channel step a lane (i = l % 16, group
// g = l / 16) loads channels 8g .. 8g + 7 of its token row and of its basis row (16-byte loads,
// no LDS), and MFMA step s takes channel 8g + s from every group.  The f64 accumulator holds
// element v of lane l at row (l / 16) + 4v, column l % 16: token g + 4v, rank i of the block.
// ---------------------------------------------------------------------------------------------

template <int DT>
__global__ void __launch_bounds__(kThreads) project_kernel(const rch_fit_matrix* __restrict__ mats, int channels) {
    const rch_fit_matrix* M = mats + blockIdx.z;
    const int64_t rows = M->rows;
    const int rank = static_cast<int>(M->rank);
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * 64;
    const int r0 = blockIdx.y * 64;
    if (t0 >= rows || r0 >= rank) return;
    constexpr int E = esize<DT>();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int g = lane >> 4, i16 = lane & 15;
    const int64_t wt = t0 + 16 * wave;  // first token of this wave
    const __amdgpu_buffer_rsrc_t xs = source_rows<DT>(M, channels, wt);
    const __amdgpu_buffer_rsrc_t qs = make_rsrc(M->basis_ptr, ((rank - 1) * M->basis_stride + channels) * 2);
    const uint32_t x_row = static_cast<uint32_t>(i16 * M->src_stride * E);

    d4 acc[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[b] = d4{};
    for (int c0 = 0; c0 < channels; c0 += 32) {
        const int c = c0 + 8 * g;
        double xv[8];
        load8<DT>(xs, c < channels ? x_row + static_cast<uint32_t>(c * E) : kOutOfRange, xv);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int k = r0 + 16 * b + i16;
            const uint32_t q_off =
                (k < rank && c < channels) ? static_cast<uint32_t>((k * M->basis_stride + c) * 2) : kOutOfRange;
            if (r0 + 16 * b >= rank) continue;  // uniform: a 16-rank block past the rank adds zeros
            double qv[8];
            load8<RCH_DT_F16>(qs, q_off, qv);
#pragma unroll
            for (int s = 0; s < 8; ++s) acc[b] = __builtin_amdgcn_mfma_f64_16x16x4f64(xv[s], qv[s], acc[b], 0, 0, 0);
        }
    }

    RCH_GLOBAL float* out = gout<float>(M->coef_ptr);
    unsigned int* ext = reinterpret_cast<unsigned int*>(M->extrema_ptr);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const int k = r0 + 16 * b + i16;  // this lane's rank
        uint32_t lo = 0u, hi = 0u;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int64_t t = wt + g + 4 * v;
            const float value = static_cast<float>(acc[b][v]);
            if (t < rows) {
                if (k < rank) out[t * M->coef_stride + k] = value;  // 16 lanes: 64 contiguous bytes of a row
                const uint32_t key = order_key(value);
                lo = ~key > lo ? ~key : lo;
                hi = key > hi ? key : hi;
            }
        }
        if (ext) {
#pragma unroll
            for (int d = 16; d <= 32; d <<= 1) {  // over the 4 token groups
                const uint32_t ol = __shfl_xor(lo, d), oh = __shfl_xor(hi, d);
                lo = ol > lo ? ol : lo;
                hi = oh > hi ? oh : hi;
            }
            if (g == 0 && k < rank) {
                atomicMax(ext + k, lo);  // vector atomics
                atomicMax(ext + rank + k, hi);
            }
        }
    }
}

// The 4 channels of tokens g + 4v (v = 0..3) of a lane's 64-channel group, as raw 16-bit pairs
// (or fp32 words), loaded ahead of their use.
template <int DT>
struct SourceQuad {
    using word = std::conditional_t<DT == RCH_DT_F32, u4, u2>;
    word w[4];
};

template <int DT>
__device__ __forceinline__ void load_quad(__amdgpu_buffer_rsrc_t xs, const rch_fit_matrix* M, int c, bool c_ok,
                                          SourceQuad<DT>& q) {
    constexpr int E = esize<DT>();
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int token = (threadIdx.x & 63) / 16 + 4 * v;
        const uint32_t offset = c_ok ? static_cast<uint32_t>((token * M->src_stride + c) * E) : kOutOfRange;
        if constexpr (DT == RCH_DT_F32) {
            q.w[v] = __builtin_amdgcn_raw_buffer_load_b128(xs, offset, 0, 0);
        } else {
            q.w[v] = __builtin_amdgcn_raw_buffer_load_b64(xs, offset, 0, 0);
        }
    }
}

// Residual of one 64-channel group: e = x - r per element, FP64 sums of x^2 and e^2, optional fp32 store.
template <int DT>
__device__ __forceinline__ void residual_group(const SourceQuad<DT>& q, const d4 (&acc)[4], int c, bool c_ok,
                                               int64_t wt, int64_t left, int channels, RCH_GLOBAL float* resid,
                                               double& src, double& err) {
    const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int token = g + 4 * v;
        double a[4];
        if constexpr (DT == RCH_DT_F32) {
#pragma unroll
            for (int b = 0; b < 4; ++b) a[b] = static_cast<double>(__uint_as_float(q.w[v][b]));
        } else {
#pragma unroll
            for (int b = 0; b < 4; ++b) a[b] = static_cast<double>(half_bits<DT>((q.w[v][b >> 1] >> (16 * (b & 1))) & 0xffffu));
        }
        double e[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            e[b] = a[b] - acc[b][v];
            // The scale s is applied once per tile: sum (a / s)^2 = (sum a^2) / s^2 up to the rounding
            // of the FP64 sums (relative 1e-16), without two FP64 divisions per element.
            src += a[b] * a[b];
            err += e[b] * e[b];
        }
        if (resid && c_ok && token < left) {
            const f4 out = {static_cast<float>(e[0]), static_cast<float>(e[1]), static_cast<float>(e[2]),
                            static_cast<float>(e[3])};
            *reinterpret_cast<RCH_GLOBAL f4*>(resid + (wt + token) * channels + c) = out;
        }
    }
}

// The four B operands (channels 4i .. 4i + 3 of basis row k) from one 8-byte load, as doubles.
__device__ __forceinline__ double basis_operand(const u2& w, int b) {
    return static_cast<double>(half_bits<RCH_DT_F16>((w[b >> 1] >> (16 * (b & 1))) & 0xffffu));
}

// ---------------------------------------------------------------------------------------------
// Residual energies on v_mfma_f64_16x16x4f64: D[m = token][n = channel] = sum_k P[token][k] Q[k][c].
// Workgroup = 64-token tile of one matrix, wave w = tokens 16w .. 16w + 15, looping over
// 64-channel groups.  A group is four 16 x 16 blocks whose columns interleave: column i of
// block b is channel 4i + b of the group, so after the four blocks lane l (i = l % 16,
// g = l / 16) holds channels 4i .. 4i + 3 of tokens g + 4v (v = 0..3, the f64 accumulator's row
// (l / 16) + 4v): X and the residual move as 4-channel vectors, 16 lanes covering 64 contiguous
// channels of a row.  Per 16-rank step a lane takes P[token i][4g .. 4g + 3] (the A operand; MFMA
// step j takes rank 4g + j) and, for each j, Q[4g + j][4i .. 4i + 3] (one 8-byte load: the B
// operands of the four blocks).
//
// Ranks up to 64 (the common fit ranks) keep the wave's P block in registers for the whole
// channel loop (loaded once instead of once per channel group) and load a group's source
// elements before its MFMAs; larger ranks stream P per step.  Both paths add the products in the same
// order (rank ascending within each block), so their results are identical.
// ---------------------------------------------------------------------------------------------

template <int DT>
__global__ void __launch_bounds__(kThreads) residual_kernel(const rch_fit_matrix* __restrict__ mats, int channels) {
    const rch_fit_matrix* M = mats + blockIdx.y;
    const int64_t rows = M->rows;
    const int rank = static_cast<int>(M->rank);
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * 64;
    if (t0 >= rows) return;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int g = lane >> 4, i16 = lane & 15;
    const int64_t wt = t0 + 16 * wave;
    const int64_t left = rows - wt;
    const __amdgpu_buffer_rsrc_t xs = source_rows<DT>(M, channels, wt);
    const __amdgpu_buffer_rsrc_t ps = make_rsrc(M->coef_ptr + wt * M->coef_stride * 4,
                                                (rank > 0 && left > 0) ? ((left - 1) * M->coef_stride + rank) * 4 : 0);
    const __amdgpu_buffer_rsrc_t qs = make_rsrc(M->basis_ptr, rank > 0 ? ((rank - 1) * M->basis_stride + channels) * 2 : 0);
    const float smax = __uint_as_float(*gin<unsigned int>(M->absmax_ptr));
    const double s = static_cast<double>(smax);
    const bool scaled = smax != 0.0f;
    const uint32_t p_row = static_cast<uint32_t>(i16 * M->coef_stride * 4);
    const uint32_t q_stride = static_cast<uint32_t>(M->basis_stride * 2);
    RCH_GLOBAL float* resid = M->resid_ptr ? gout<float>(M->resid_ptr) : nullptr;

    double src = 0.0, err = 0.0;
    if (rank <= 64) {
        const int steps = (rank + 15) >> 4;  // uniform
        u4 pw[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int k = 16 * t + 4 * g;
            pw[t] = __builtin_amdgcn_raw_buffer_load_b128(ps, (t < steps && k < rank) ? p_row + static_cast<uint32_t>(k * 4)
                                                                                     : kOutOfRange, 0, 0);
        }
        for (int c64 = 0; c64 < channels; c64 += 64) {
            const int c = c64 + 4 * i16;  // this lane's 4 channels (channels % 8 == 0: all or none in range)
            const bool c_ok = c < channels;
            SourceQuad<DT> xq;
            load_quad<DT>(xs, M, c, c_ok, xq);
            d4 acc[4] = {d4{}, d4{}, d4{}, d4{}};
#pragma unroll 1
            for (int t = 0; t < steps; ++t) {
                const int k = 16 * t + 4 * g;
                u2 qw[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t q_off =
                        (k + j < rank && c_ok) ? static_cast<uint32_t>(k + j) * q_stride + 2u * c : kOutOfRange;
                    qw[j] = __builtin_amdgcn_raw_buffer_load_b64(qs, q_off, 0, 0);
                }
                const u4 p = t == 0 ? pw[0] : t == 1 ? pw[1] : t == 2 ? pw[2] : pw[3];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    // P rows may hold padding beyond the rank; its basis rows read as zero.
                    const double pa = k + j < rank ? static_cast<double>(__uint_as_float(p[j])) : 0.0;
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        acc[b] = __builtin_amdgcn_mfma_f64_16x16x4f64(pa, basis_operand(qw[j], b), acc[b], 0, 0, 0);
                }
            }
            residual_group<DT>(xq, acc, c, c_ok, wt, left, channels, resid, src, err);
        }
    } else {
        for (int c64 = 0; c64 < channels; c64 += 64) {
            const int c = c64 + 4 * i16;
            const bool c_ok = c < channels;
            d4 acc[4] = {d4{}, d4{}, d4{}, d4{}};
            for (int k0 = 0; k0 < rank; k0 += 16) {
                const int k = k0 + 4 * g;
                const u4 pw = __builtin_amdgcn_raw_buffer_load_b128(
                    ps, k < rank ? p_row + static_cast<uint32_t>(k * 4) : kOutOfRange, 0, 0);
                u2 qw[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t q_off =
                        (k + j < rank && c_ok) ? static_cast<uint32_t>(k + j) * q_stride + 2u * c : kOutOfRange;
                    qw[j] = __builtin_amdgcn_raw_buffer_load_b64(qs, q_off, 0, 0);
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const double pa = k + j < rank ? static_cast<double>(__uint_as_float(pw[j])) : 0.0;
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        acc[b] = __builtin_amdgcn_mfma_f64_16x16x4f64(pa, basis_operand(qw[j], b), acc[b], 0, 0, 0);
                }
            }
            SourceQuad<DT> xq;
            load_quad<DT>(xs, M, c, c_ok, xq);
            residual_group<DT>(xq, acc, c, c_ok, wt, left, channels, resid, src, err);
        }
    }
    // Fixed-order reduction: butterfly within the wave, then waves 0..3 in order.
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        src += __shfl_xor(src, d);
        err += __shfl_xor(err, d);
    }
    __shared__ double part[2][kThreads / 64];
    if (lane == 0) {
        part[0][wave] = src;
        part[1][wave] = err;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double a = 0.0, b = 0.0;
        for (int w = 0; w < kThreads / 64; ++w) {
            a += part[0][w];
            b += part[1][w];
        }
        if (scaled) {
            a = a / s / s;
            b = b / s / s;
        }
        RCH_GLOBAL double* out = gout<double>(M->partial_ptr) + 2 * blockIdx.x;
        out[0] = a;
        out[1] = b;
    }
}

// Sum of the per-tile partials of each matrix in tile order (one workgroup per matrix).
__global__ void __launch_bounds__(64) energy_total_kernel(const rch_fit_matrix* __restrict__ mats) {
    const rch_fit_matrix* M = mats + blockIdx.x;
    if (threadIdx.x != 0) return;
    const int64_t tiles = (M->rows + 63) / 64;
    const RCH_GLOBAL double* p = gin<double>(M->partial_ptr);
    double a = 0.0, b = 0.0;
    for (int64_t t = 0; t < tiles; ++t) {
        a += p[2 * t];
        b += p[2 * t + 1];
    }
    RCH_GLOBAL double* out = gout<double>(M->energy_ptr);
    out[0] = a;
    out[1] = b;
}

// ---------------------------------------------------------------------------------------------
// Column extrema and the FP64 quantizer of an fp32 [rows, cols] matrix: workgroup = 64 rows,
// threads stride over the columns (consecutive threads, consecutive columns).
// ---------------------------------------------------------------------------------------------

__global__ void __launch_bounds__(kThreads) extrema_kernel(const float* __restrict__ values, int64_t rows, int cols,
                                                           int64_t stride, unsigned int* __restrict__ keys) {
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * 64;
    const int64_t r1 = rows - r0 < 64 ? rows : r0 + 64;
    for (int c = threadIdx.x; c < cols; c += kThreads) {
        uint32_t lo = 0u, hi = 0u;
        for (int64_t r = r0; r < r1; ++r) {
            const uint32_t k = order_key(values[r * stride + c]);
            lo = ~k > lo ? ~k : lo;
            hi = k > hi ? k : hi;
        }
        atomicMax(keys + c, lo);  // vector atomics
        atomicMax(keys + cols + c, hi);
    }
}

__global__ void __launch_bounds__(kThreads) quantize_kernel(const float* __restrict__ values, int64_t rows, int cols,
                                                            int64_t stride, const double* __restrict__ scale,
                                                            const double* __restrict__ offset,
                                                            uint8_t* __restrict__ codes, int64_t code_stride) {
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * 64;
    const int64_t r1 = rows - r0 < 64 ? rows : r0 + 64;
    for (int c = threadIdx.x; c < cols; c += kThreads) {
        const double sc = scale[c], of = offset[c];
        for (int64_t r = r0; r < r1; ++r) {
            double q = 0.0;
            if (sc > 0.0) q = rint((static_cast<double>(values[r * stride + c]) - of) / sc);
            q = q < 0.0 ? 0.0 : (q > 255.0 ? 255.0 : q);
            codes[r * code_stride + c] = static_cast<uint8_t>(q);
        }
    }
}

__global__ void __launch_bounds__(kThreads) quantize_batched_kernel(const rch_quantize_job* __restrict__ jobs) {
    const rch_quantize_job* J = jobs + blockIdx.y;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * 64;
    if (r0 >= J->rows) return;
    const int64_t r1 = J->rows - r0 < 64 ? J->rows : r0 + 64;
    const int cols = static_cast<int>(J->cols);
    const RCH_GLOBAL float* values = gin<float>(J->values_ptr);
    const RCH_GLOBAL double* affine = gin<double>(J->affine_ptr);
    RCH_GLOBAL uint8_t* codes = gout<uint8_t>(J->codes_ptr);
    for (int c = threadIdx.x; c < cols; c += kThreads) {
        const double sc = affine[c], of = affine[cols + c];
        for (int64_t r = r0; r < r1; ++r) {
            double q = 0.0;
            if (sc > 0.0) q = rint((static_cast<double>(values[r * J->stride + c]) - of) / sc);
            q = q < 0.0 ? 0.0 : (q > 255.0 ? 255.0 : q);
            codes[r * J->code_stride + c] = static_cast<uint8_t>(q);
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Batched FP64 Cholesky factor and triangular inverse (the planner's CholeskyQR steps): one
// 1024-thread workgroup per k x k matrix, whose upper triangle lives in LDS in packed row-major
// form, with one workgroup barrier per factor column and one per inverse row.
//
// Factorization (right-looking): in step j every thread reads the pivot d = A[j][j], forms
// 1 / sqrt(d) itself and applies the rank-1 update A[i][c] -= (A[j][i] / r)(A[j][c] / r) to its
// share of the trailing triangle j < i <= c, reading row j unscaled (no thread writes row j in
// step j).  The scaled row j = row j of R goes to a row buffer and is written back into the
// triangle in step j + 1, when no thread reads row j.
//
// Inverse X = R^-1, rows from the bottom: S[r][c] accumulates sum_{p > r} R[r][p] X[p][c] as rows
// p are finished.  In step i, row i is final: X[i][c] = (delta_ic - S[i][c]) / R[i][i]; every
// thread forms the values of row i it needs from S[i][c] and adds R[r][i] X[i][c] into S[r][c]
// for its share of r < i <= c.  Row i of X goes to a row buffer and replaces row i of S in step
// i - 1.  Lanes run over columns and waves over rows, so a wave's LDS accesses are one row of
// consecutive doubles plus one broadcast word.
// ---------------------------------------------------------------------------------------------

constexpr int kCholThreads = 1024;
constexpr int kCholWaves = kCholThreads / 64;
constexpr int kCholPacked = RCH_CHOLESKY_MAX_K * (RCH_CHOLESKY_MAX_K + 1) / 2;

// Offset of (i, c), i <= c, in a packed upper triangle of order k (rows i = 0.. stored back to back).
__device__ __forceinline__ int packed_at(int i, int c, int k) { return i * k - (i * (i - 1)) / 2 + (c - i); }

__global__ void __launch_bounds__(kCholThreads) cholesky_inverse_kernel(const double* __restrict__ a,
                                                                         double* __restrict__ x,
                                                                         int32_t* __restrict__ info, int k) {
    __shared__ double m[kCholPacked];   // A, then R (off-diagonal; the diagonal keeps the pivots)
    __shared__ double s[kCholPacked];   // S, then X
    __shared__ double rowbuf[2][RCH_CHOLESKY_MAX_K];
    __shared__ double diag[RCH_CHOLESKY_MAX_K];  // 1 / R[j][j]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t base = static_cast<int64_t>(blockIdx.x) * k * k;
    const RCH_GLOBAL double* A = gin<double>(reinterpret_cast<int64_t>(a)) + base;
    RCH_GLOBAL double* X = gout<double>(reinterpret_cast<int64_t>(x)) + base;
    for (int i = wave; i < k; i += kCholWaves) {
        for (int c = i + lane; c < k; c += 64) {
            m[packed_at(i, c, k)] = A[i * k + c];
            s[packed_at(i, c, k)] = 0.0;
        }
    }
    __syncthreads();
    int failed = 0;
    for (int j = 0; j < k; ++j) {
        const double d = m[packed_at(j, j, k)];  // every thread reads the same pivot: the branch is uniform
        if (!(d > 0.0) || !(d < INFINITY)) {
            failed = j + 1;
            break;
        }
        const double inv = 1.0 / sqrt(d);
        if (j > 0) {  // row j - 1 of R, scaled in the previous step
            for (int c = j + tid; c < k; c += kCholThreads) m[packed_at(j - 1, c, k)] = rowbuf[(j - 1) & 1][c];
        }
        const int row_j = packed_at(j, j, k) - j;  // row j's entry c sits at row_j + c
        for (int c = j + 1 + tid; c < k; c += kCholThreads) rowbuf[j & 1][c] = m[row_j + c] * inv;
        if (tid == 0) diag[j] = inv;
        for (int i = j + 1 + wave; i < k; i += kCholWaves) {
            const double ri = m[row_j + i] * inv;
            const int row_i = packed_at(i, i, k) - i;
            for (int c = i + lane; c < k; c += 64) {
                const double rc = m[row_j + c] * inv;
                const double product = ri * rc;
                m[row_i + c] = m[row_i + c] - product;
            }
        }
        __syncthreads();
    }
    if (failed) {
        for (int i = wave; i < k; i += kCholWaves)
            for (int c = lane; c < k; c += 64) X[i * k + c] = i == c ? 1.0 : 0.0;
        if (tid == 0) info[blockIdx.x] = failed;
        return;
    }
    // Step k - 1 wrote row k - 2 back and row k - 1 has no off-diagonal entry: m holds R above
    // the diagonal (the last step's barrier makes it visible).
    for (int i = k - 1; i >= 0; --i) {
        const double di = diag[i];
        const int srow_i = packed_at(i, i, k) - i;
        if (i + 1 < k) {  // row i + 1 of X, finished in the previous step
            for (int c = i + 1 + tid; c < k; c += kCholThreads) s[packed_at(i + 1, c, k)] = rowbuf[(i + 1) & 1][c];
        }
        for (int c = i + tid; c < k; c += kCholThreads) rowbuf[i & 1][c] = ((c == i ? 1.0 : 0.0) - s[srow_i + c]) * di;
        for (int r = wave; r < i; r += kCholWaves) {
            const double rri = m[packed_at(r, i, k)];
            const int srow_r = packed_at(r, r, k) - r;
            for (int c = i + lane; c < k; c += 64) {
                const double xic = ((c == i ? 1.0 : 0.0) - s[srow_i + c]) * di;
                const double product = rri * xic;
                s[srow_r + c] = s[srow_r + c] + product;
            }
        }
        __syncthreads();
    }
    for (int c = tid; c < k; c += kCholThreads) s[packed_at(0, c, k)] = rowbuf[0][c];
    __syncthreads();
    for (int i = wave; i < k; i += kCholWaves)
        for (int c = lane; c < k; c += 64) X[i * k + c] = i <= c ? s[packed_at(i, c, k)] : 0.0;
    if (tid == 0) info[blockIdx.x] = 0;
}

// ---------------------------------------------------------------------------------------------
// Seeded Gaussian columns (start blocks of the subspace solvers)
//
// Counter-based Philox-4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as
// 1, 2, 3", SC 2011): the key is the job's 64-bit seed, the counter the index of a group of four
// elements, so every element has a fixed value whatever the launch shape.  Box-Muller turns each
// pair of 32-bit words into two standard normals.
// ---------------------------------------------------------------------------------------------

__device__ __forceinline__ void philox4x32_10(uint32_t (&c)[4], uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int round = 0; round < 10; ++round) {
        const uint64_t p0 = static_cast<uint64_t>(0xD2511F53u) * c[0];
        const uint64_t p1 = static_cast<uint64_t>(0xCD9E8D57u) * c[2];
        const uint32_t hi0 = static_cast<uint32_t>(p0 >> 32), lo0 = static_cast<uint32_t>(p0);
        const uint32_t hi1 = static_cast<uint32_t>(p1 >> 32), lo1 = static_cast<uint32_t>(p1);
        c[0] = hi1 ^ c[1] ^ k0;
        c[1] = lo1;
        c[2] = hi0 ^ c[3] ^ k1;
        c[3] = lo0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}

__global__ void __launch_bounds__(256) gaussian_kernel(const rch_gauss_job* __restrict__ jobs) {
    const rch_gauss_job& J = jobs[blockIdx.y];
    const int64_t total = J.rows * J.cols;
    const int64_t group = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // elements 4 group .. + 3
    if (4 * group >= total) return;
    uint32_t c[4] = {static_cast<uint32_t>(group), static_cast<uint32_t>(group >> 32), 0u, 0u};
    philox4x32_10(c, static_cast<uint32_t>(J.seed), static_cast<uint32_t>(static_cast<uint64_t>(J.seed) >> 32));
    float z[4];
#pragma unroll
    for (int pair = 0; pair < 2; ++pair) {
        // Uniforms in (0, 1]: (word + 1) * 2^-32 keeps log away from zero.
        const float u1 = (static_cast<float>(c[2 * pair]) + 1.0f) * 2.3283064365386963e-10f;
        const float u2 = static_cast<float>(c[2 * pair + 1]) * 2.3283064365386963e-10f;
        const float r = sqrtf(-2.0f * logf(u1));
        z[2 * pair] = r * cosf(6.283185307179586f * u2);
        z[2 * pair + 1] = r * sinf(6.283185307179586f * u2);
    }
    RCH_GLOBAL float* dst = gout<float>(J.dst_ptr);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t e = 4 * group + i;
        if (e < total) {
            const int64_t r = e / J.cols, col = e - r * J.cols;
            dst[r * J.stride + col] = z[i];
        }
    }
}

int check_matrices(const rch_fit_matrix* mats, int n, int channels, const char* what) {
    if (!mats || n <= 0 || n > 65535) return fail(RCH_E_CONFIG, "%s: 1 <= n_mats <= 65535 required", what);
    if (channels <= 0 || channels % 8 != 0 || channels > (1 << 20))
        return fail(RCH_E_CONFIG, "%s: channels must be a positive multiple of 8", what);
    return RCH_OK;
}

}  // namespace
}  // namespace rch

using namespace rch;

#define RCH_DISPATCH_DTYPE_BLOCK(dtype, what, KERNEL, GRID, BLOCK, ...)                                             \
    switch (dtype) {                                                                                                \
        case RCH_DT_BF16: hipLaunchKernelGGL(KERNEL<RCH_DT_BF16>, GRID, dim3(BLOCK), 0, s, __VA_ARGS__); break;     \
        case RCH_DT_F16: hipLaunchKernelGGL(KERNEL<RCH_DT_F16>, GRID, dim3(BLOCK), 0, s, __VA_ARGS__); break;       \
        case RCH_DT_F32: hipLaunchKernelGGL(KERNEL<RCH_DT_F32>, GRID, dim3(BLOCK), 0, s, __VA_ARGS__); break;       \
        default: return fail(RCH_E_CONFIG, "%s: source dtype must be bf16, f16 or f32", what);                      \
    }
#define RCH_DISPATCH_DTYPE(dtype, what, KERNEL, GRID, ...) \
    RCH_DISPATCH_DTYPE_BLOCK(dtype, what, KERNEL, GRID, kThreads, __VA_ARGS__)

extern "C" {

int rch_fit_matrix_size(void) { return static_cast<int>(sizeof(rch_fit_matrix)); }

int rch_fit_absmax(const rch_fit_matrix* mats_dev, int n_mats, int channels, int64_t max_rows, int src_dtype,
                   void* stream) {
    if (int status = check_matrices(mats_dev, n_mats, channels, "rch_fit_absmax")) return status;
    if (max_rows <= 0 || (max_rows + 63) / 64 > 0x7fffffff) return fail(RCH_E_CONFIG, "rch_fit_absmax: invalid max_rows");
    const dim3 grid(static_cast<unsigned>((max_rows + 63) / 64), static_cast<unsigned>(n_mats));
    hipStream_t s = as_stream(stream);
    RCH_DISPATCH_DTYPE(src_dtype, "rch_fit_absmax", absmax_kernel, grid, mats_dev, channels);
    return check_launch("rch_fit_absmax");
}

int rch_fit_gram(const rch_fit_matrix* mats_dev, int n_mats, int channels, int src_dtype, void* stream) {
    if (int status = check_matrices(mats_dev, n_mats, channels, "rch_fit_gram")) return status;
    const int t = (channels + kGramTile - 1) / kGramTile;
    const int64_t tiles = static_cast<int64_t>(t) * (t + 1) / 2;
    if (tiles * n_mats > 0x7fffffff) return fail(RCH_E_CONFIG, "rch_fit_gram: too many tiles");
    const int grid = static_cast<int>(tiles * n_mats);
    hipStream_t s = as_stream(stream);
    RCH_DISPATCH_DTYPE_BLOCK(src_dtype, "rch_fit_gram", gram_kernel, dim3(grid), kGramThreads, mats_dev, channels,
                             static_cast<int>(tiles), grid);
    return check_launch("rch_fit_gram");
}

int rch_fit_project(const rch_fit_matrix* mats_dev, int n_mats, int channels, int64_t max_rows, int max_rank,
                    int src_dtype, void* stream) {
    if (int status = check_matrices(mats_dev, n_mats, channels, "rch_fit_project")) return status;
    if (max_rows <= 0 || max_rank <= 0 || (max_rows + 63) / 64 > 0x7fffffff || max_rank > channels)
        return fail(RCH_E_CONFIG, "rch_fit_project: invalid max_rows / max_rank");
    const dim3 grid(static_cast<unsigned>((max_rows + 63) / 64), static_cast<unsigned>((max_rank + 63) / 64),
                    static_cast<unsigned>(n_mats));
    hipStream_t s = as_stream(stream);
    RCH_DISPATCH_DTYPE(src_dtype, "rch_fit_project", project_kernel, grid, mats_dev, channels);
    return check_launch("rch_fit_project");
}

int rch_fit_residual(const rch_fit_matrix* mats_dev, int n_mats, int channels, int64_t max_rows, int src_dtype,
                     void* stream) {
    if (int status = check_matrices(mats_dev, n_mats, channels, "rch_fit_residual")) return status;
    if (max_rows <= 0 || (max_rows + 63) / 64 > 0x7fffffff) return fail(RCH_E_CONFIG, "rch_fit_residual: invalid max_rows");
    const dim3 grid(static_cast<unsigned>((max_rows + 63) / 64), static_cast<unsigned>(n_mats));
    hipStream_t s = as_stream(stream);
    RCH_DISPATCH_DTYPE(src_dtype, "rch_fit_residual", residual_kernel, grid, mats_dev, channels);
    if (int status = check_launch("rch_fit_residual")) return status;
    hipLaunchKernelGGL(energy_total_kernel, dim3(n_mats), dim3(64), 0, s, mats_dev);
    return check_launch("rch_fit_residual (totals)");
}

int rch_column_extrema(const float* values_dev, int64_t rows, int cols, int64_t stride, uint32_t* keys_dev,
                       void* stream) {
    if (!values_dev || !keys_dev || rows <= 0 || cols <= 0 || stride < cols || (rows + 63) / 64 > 0x7fffffff)
        return fail(RCH_E_CONFIG, "rch_column_extrema: invalid arguments");
    hipLaunchKernelGGL(extrema_kernel, dim3(static_cast<unsigned>((rows + 63) / 64)), dim3(kThreads), 0,
                       as_stream(stream), values_dev, rows, cols, stride, reinterpret_cast<unsigned int*>(keys_dev));
    return check_launch("rch_column_extrema");
}

int rch_quantize(const float* values_dev, int64_t rows, int cols, int64_t stride, const double* scale_dev,
                 const double* offset_dev, uint8_t* codes_dev, int64_t code_stride, void* stream) {
    if (!values_dev || !scale_dev || !offset_dev || !codes_dev || rows <= 0 || cols <= 0 || stride < cols ||
        code_stride < cols || (rows + 63) / 64 > 0x7fffffff)
        return fail(RCH_E_CONFIG, "rch_quantize: invalid arguments");
    hipLaunchKernelGGL(quantize_kernel, dim3(static_cast<unsigned>((rows + 63) / 64)), dim3(kThreads), 0,
                       as_stream(stream), values_dev, rows, cols, stride, scale_dev, offset_dev, codes_dev, code_stride);
    return check_launch("rch_quantize");
}

int rch_cholesky_inverse(const double* a_dev, double* x_dev, int32_t* info_dev, int n, int k, void* stream) {
    if (!a_dev || !x_dev || !info_dev || n <= 0 || k <= 0 || k > RCH_CHOLESKY_MAX_K)
        return fail(RCH_E_CONFIG, "rch_cholesky_inverse: 1 <= k <= %d and device buffers required", RCH_CHOLESKY_MAX_K);
    hipLaunchKernelGGL(cholesky_inverse_kernel, dim3(static_cast<unsigned>(n)), dim3(kCholThreads), 0, as_stream(stream),
                       a_dev, x_dev, info_dev, k);
    return check_launch("rch_cholesky_inverse");
}

int rch_fit_gaussian(const rch_gauss_job* jobs_dev, int n_jobs, int64_t max_elements, void* stream) {
    if (!jobs_dev || n_jobs <= 0 || n_jobs > 65535 || max_elements <= 0 || (max_elements + 1023) / 1024 > 0x7fffffff)
        return fail(RCH_E_CONFIG, "rch_fit_gaussian: invalid arguments");
    const dim3 grid(static_cast<unsigned>((max_elements + 1023) / 1024), static_cast<unsigned>(n_jobs));
    hipLaunchKernelGGL(gaussian_kernel, grid, dim3(256), 0, as_stream(stream), jobs_dev);
    return check_launch("rch_fit_gaussian");
}

int rch_quantize_batched(const rch_quantize_job* jobs_dev, int n_jobs, int64_t max_rows, void* stream) {
    if (!jobs_dev || n_jobs <= 0 || n_jobs > 65535 || max_rows <= 0 || (max_rows + 63) / 64 > 0x7fffffff)
        return fail(RCH_E_CONFIG, "rch_quantize_batched: invalid arguments");
    const dim3 grid(static_cast<unsigned>((max_rows + 63) / 64), static_cast<unsigned>(n_jobs));
    hipLaunchKernelGGL(quantize_batched_kernel, grid, dim3(kThreads), 0, as_stream(stream), jobs_dev);
    return check_launch("rch_quantize_batched");
}

}  // extern "C"
