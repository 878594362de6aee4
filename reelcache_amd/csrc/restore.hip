// Restore entry points for MI355X (gfx950): basis packing, coefficient bounds, the dense
// RoPE store, and dispatch of the fused restore kernel (restore_kernel.h).
//
// Reference: reelcache/restore_kernels.py (_bound_kernel :1588-1606, _rope_store_kernel
// :1557-1585, _fused_group / _two_pass_group :2025-2121).
#include <mutex>

#include "restore_fast.h"
#include "restore_stream.h"

namespace rch {
namespace {

// ---------------------------------------------------------------------------------------------
// Basis packing
// ---------------------------------------------------------------------------------------------

// Eight consecutive channels c .. c + 7 of basis row r as floats (zero beyond the channels).
// `vec`: 16-byte aligned rows of 16-bit values (one load), else element loads.
__device__ __forceinline__ void basis_row8(const rch_pack& P, int dtype, bool vec, int64_t r, int64_t c, float (&v)[8]) {
    const int64_t base = r * P.row_stride + c;
    if (vec && c + 8 <= P.channels) {
        const u4 raw = *reinterpret_cast<const RCH_GLOBAL u4*>(P.src_ptr + 2 * base);
        if (dtype == RCH_DT_F16) {
            const h8 x = __builtin_bit_cast(h8, raw);
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = static_cast<float>(x[j]);
        } else {
            const bf8 x = __builtin_bit_cast(bf8, raw);
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = static_cast<float>(x[j]);
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = c + j < P.channels ? load_value(P.src_ptr, base + j, dtype) : 0.0f;
}

// Max pass of a pack workgroup: max|Q| over rows row_lane + 32 u (all u with a row below the
// rank) of the thread's 8 channels c .. c + 7, keeping row stage_row in stage.  Eight rows per
// thread are in flight together (one pass up to rank 256); rows past the rank re-read the last
// row (a duplicate does not change the maximum).  VEC: 16-byte aligned f16 / bf16 rows and a
// channel count that is a multiple of 8, loaded as one 16-byte word per row with no branch
// between the loads; else element loads.
template <bool VEC>
__device__ __forceinline__ float pack_max(const rch_pack& P, int dtype, int64_t c, int row_lane, int64_t stage_row,
                                          float (&stage)[8]) {
    constexpr int kRows = 8;
    const bool in = c < P.channels;
    const bool staged = stage_row < P.rank;
    float m = 0.0f;
    for (int64_t r0 = row_lane; r0 < P.rank; r0 += 32 * kRows) {
        float v[kRows][8];
        if constexpr (VEC) {
            u4 raw[kRows];
#pragma unroll
            for (int u = 0; u < kRows; ++u) {
                const int64_t r = min(r0 + 32 * u, P.rank - 1);
                raw[u] = in ? *reinterpret_cast<const RCH_GLOBAL u4*>(P.src_ptr + 2 * (r * P.row_stride + c)) : u4{0u, 0u, 0u, 0u};
            }
            if (dtype == RCH_DT_F16) {
#pragma unroll
                for (int u = 0; u < kRows; ++u) {
                    const h8 x = __builtin_bit_cast(h8, raw[u]);
#pragma unroll
                    for (int j = 0; j < 8; ++j) v[u][j] = static_cast<float>(x[j]);
                }
            } else {
#pragma unroll
                for (int u = 0; u < kRows; ++u) {
                    const bf8 x = __builtin_bit_cast(bf8, raw[u]);
#pragma unroll
                    for (int j = 0; j < 8; ++j) v[u][j] = static_cast<float>(x[j]);
                }
            }
        } else {
#pragma unroll
            for (int u = 0; u < kRows; ++u) basis_row8(P, dtype, false, min(r0 + 32 * u, P.rank - 1), c, v[u]);
        }
#pragma unroll
        for (int u = 0; u < kRows; ++u) {
            const bool mine = staged && r0 + 32 * u == stage_row;  // never a clamped re-read
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                m = fmaxf(m, fabsf(v[u][j]));
                stage[j] = mine ? v[u][j] : stage[j];
            }
        }
    }
    return m;
}

// Packs rows Q[:rank] of each basis into MFMA A-operand fragments.  Workgroup (g, sp, p) owns
// 32-channel blocks 2g, 2g + 1 and 16-row steps 2sp, 2sp + 1 of basis p.  Fragment (s, nb, lane)
// holds Q[16 s + k_slot(h, j), 32 nb + block_channel(lane % 32)] for j = 0..7 (h = lane / 32).
// Fp16 fragments of a non-fp16 basis are prescaled by 2**e per 32-channel block so that the
// block's max|Q| lands in (2**13, 2**14] (exact powers of two; e is written to exps[nb] and
// undone by the restore epilogue).  Every workgroup reduces the max of its blocks itself
// (rows are re-read from L2), so one launch suffices; its own staged rows come from the same
// loads, so the workgroup makes one round of global reads (up to rank 256).
// A workgroup writes the stream kernel's slabs of four 32-channel blocks of pack P (one per wave).
// Lane (h, rho) of a wave holds channel 32 nb + block_channel(rho) and ranks 16 s + 8 h + j of
// W = s_k Q_kc.  The block's exponent e puts max|W| in (2**13, 2**14]; 2^e W is split into fp16
// hi + lo (the hi fragments of all steps, then the lo fragments); the bias
// b_c = sum_k (o_k + 128 s_k) Q_kc is summed in FP64 and rounded once.  Ranks at or beyond P.rank
// get W = 0 (the kernel multiplies arbitrary code bytes there).  The affine goes through LDS
// (shared by the four waves); every basis load of a wave is issued before the first use.
template <int KS, int DT>
__device__ __forceinline__ void stream_slab_group(const rch_pack& P) {
    __shared__ __attribute__((aligned(16))) float affine[2][16 * KS];
    const int tid = threadIdx.x;
    const int rank = static_cast<int>(P.rank);
    for (int k = tid; k < 16 * KS; k += 256) {
        affine[0][k] = k < rank ? gin<float>(P.scale_ptr)[k] : 0.0f;
        affine[1][k] = k < rank ? gin<float>(P.offset_ptr)[k] : 0.0f;
    }
    __syncthreads();
    const int64_t nb = 4 * static_cast<int64_t>(blockIdx.x) + (tid >> 6);
    if (nb >= P.nblocks) return;
    const int lane = tid & 63, h = lane >> 5, rho = lane & 31;
    const int64_t c = 32 * nb + block_channel(rho);
    const bool in = c < P.channels;
    const int64_t stride = P.row_stride;
    float w[KS][8];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int k = 16 * s + 8 * h + j;
            const bool live = in && k < rank;
            const int64_t at = live ? static_cast<int64_t>(k) * stride + c : 0;
            float q;
            if constexpr (DT == RCH_DT_F32) q = gin<float>(P.src_ptr)[at];
            else if constexpr (DT == RCH_DT_F16) q = static_cast<float>(gin<_Float16>(P.src_ptr)[at]);
            else q = static_cast<float>(gin<__bf16>(P.src_ptr)[at]);
            w[s][j] = live ? q : 0.0f;
        }
    }
    float m = 0.0f;
    double partial = 0.0;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        const int k0 = 16 * s + 8 * h;
        const f4 s0 = *reinterpret_cast<const f4*>(&affine[0][k0]), s1 = *reinterpret_cast<const f4*>(&affine[0][k0 + 4]);
        const f4 o0 = *reinterpret_cast<const f4*>(&affine[1][k0]), o1 = *reinterpret_cast<const f4*>(&affine[1][k0 + 4]);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float sc = j < 4 ? s0[j] : s1[j - 4];
            const float of = j < 4 ? o0[j] : o1[j - 4];
            partial += (static_cast<double>(of) + 128.0 * static_cast<double>(sc)) * static_cast<double>(w[s][j]);
            w[s][j] = __fmul_rn(sc, w[s][j]);
            m = fmaxf(m, fabsf(w[s][j]));
        }
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
    const int e = prescale_exponent(m);
    const float pre = pow2f(e);
    const int64_t slab = P.dst_ptr + nb * stream_slab_bytes(KS);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        h8 hi, lo;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float v = __fmul_rn(w[s][j], pre);  // exact power-of-two scale
            const _Float16 head = static_cast<_Float16>(v);
            hi[j] = head;
            lo[j] = static_cast<_Float16>(v - static_cast<float>(head));  // v - hi is exact
        }
        gout<h8>(slab)[s * 64 + lane] = hi;
        gout<h8>(slab)[(KS + s) * 64 + lane] = lo;
    }
    partial += __shfl_xor(partial, 32);
    if (h == 0) gout<float>(slab + KS * 2048)[block_channel(rho)] = static_cast<float>(partial);
    if (lane == 0) gout<int32_t>(slab + KS * 2048 + 128)[0] = e;
}

// The slab depths the stream kernel is compiled for (restore_stream.hip); slabs of any other depth
// are neither written nor read.
__host__ __device__ constexpr bool stream_pack_steps(int64_t steps) {
    return steps == 4 || steps == 8 || steps == 12 || steps == 16;
}

template <int DT>
__device__ __forceinline__ void stream_slab_steps(const rch_pack& P, int steps) {
    switch (steps) {
        case 4: stream_slab_group<4, DT>(P); break;
        case 8: stream_slab_group<8, DT>(P); break;
        case 12: stream_slab_group<12, DT>(P); break;
        case 16: stream_slab_group<16, DT>(P); break;
        default: break;  // refused: no slab is written past what the caller sized
    }
}

template <int PREC>
__device__ __forceinline__ void basis_pack_body(const rch_pack P) {
    if (P.kind == RCH_PACK_STREAM) {
        // Four blocks per workgroup, one per wave; only the y == 0 row of the grid.
        if (blockIdx.y != 0 || 4 * static_cast<int64_t>(blockIdx.x) >= P.nblocks || !stream_pack_steps(P.ksteps))
            return;
        const int steps = static_cast<int>(P.ksteps);
        switch (static_cast<int>(P.src_dtype)) {
            case RCH_DT_F32: stream_slab_steps<RCH_DT_F32>(P, steps); break;
            case RCH_DT_F16: stream_slab_steps<RCH_DT_F16>(P, steps); break;
            default: stream_slab_steps<RCH_DT_BF16>(P, steps); break;
        }
        return;
    }
    const int64_t nb0 = 2 * static_cast<int64_t>(blockIdx.x);
    const int64_t s0 = 2 * static_cast<int64_t>(blockIdx.y);
    if (nb0 >= P.nblocks || s0 >= P.ksteps) return;  // whole workgroup
    const int tid = threadIdx.x;
    const int dtype = static_cast<int>(P.src_dtype);
    const bool vec = (dtype == RCH_DT_F16 || dtype == RCH_DT_BF16) && P.src_ptr % 16 == 0 && (P.row_stride * 2) % 16 == 0;
    const bool scaled = (PREC == RCH_PREC_FP16 || PREC == RCH_PREC_FP16X2) && dtype != RCH_DT_F16;
    const int64_t c_base = 32 * nb0;  // first of the 64 channels
    // Thread layout for row loads: 32 rows x 8 chunks of 8 channels.
    const int row_lane = tid >> 3, chunk = tid & 7;
    __shared__ float tile[32][64 + 4];
    __shared__ float block_max[4][2];
    __shared__ int block_exp[2];
    // Row 16 s0 + row_lane of the 64 channels (zero beyond the rank): the row this thread stages.
    // 16 s0 = 32 blockIdx.y, so it is one of the rows row_lane + 32 u the max pass reads.
    const int64_t stage_row = 16 * s0 + row_lane;
    float stage[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) stage[j] = 0.0f;
    if (scaled) {
        const bool fast = vec && P.channels % 8 == 0;
        float m = fast ? pack_max<true>(P, dtype, c_base + 8 * chunk, row_lane, stage_row, stage)
                       : pack_max<false>(P, dtype, c_base + 8 * chunk, row_lane, stage_row, stage);
        // Block of this thread: chunk / 4.  Reduce over chunk bits 0-1 and the 8 row lanes of the wave.
        m = fmaxf(m, __shfl_xor(m, 1));
        m = fmaxf(m, __shfl_xor(m, 2));
        m = fmaxf(m, __shfl_xor(m, 8));
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));
        if ((tid & 63) == 0) block_max[tid >> 6][0] = m;
        if ((tid & 63) == 4) block_max[tid >> 6][1] = m;
#pragma unroll
        for (int j = 0; j < 8; ++j) tile[row_lane][8 * chunk + j] = stage[j];
        __syncthreads();
        if (tid < 2) {
            const float b = fmaxf(fmaxf(block_max[0][tid], block_max[1][tid]), fmaxf(block_max[2][tid], block_max[3][tid]));
            block_exp[tid] = prescale_exponent(b);
        }
    } else {
        if (stage_row < P.rank) basis_row8(P, dtype, vec, stage_row, c_base + 8 * chunk, stage);
#pragma unroll
        for (int j = 0; j < 8; ++j) tile[row_lane][8 * chunk + j] = stage[j];
        if (tid < 2) block_exp[tid] = 0;
    }
    __syncthreads();
    if (blockIdx.y == 0 && tid < 2 && nb0 + tid < P.nblocks) gout<int32_t>(P.exp_ptr)[nb0 + tid] = block_exp[tid];
    // Thread -> fragment: step s0 + (tid / 128), block nb0 + (tid / 64) % 2, lane tid % 64.
    const int sl = tid >> 7, b = (tid >> 6) & 1, lane = tid & 63, h = lane >> 5;
    const int64_t s = s0 + sl, nb = nb0 + b;
    if (s >= P.ksteps || nb >= P.nblocks) return;
    const int col = 32 * b + block_channel(lane & 31);
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = tile[16 * sl + k_slot<PREC>(h, j)][col];
    const int64_t q = (s * P.nblocks + nb) * 64 + lane;
    if constexpr (PREC == RCH_PREC_FP32) {
        RCH_GLOBAL f4* dst = gout<f4>(P.dst_ptr) + 2 * q;
        dst[0] = f4{v[0], v[1], v[2], v[3]};
        dst[1] = f4{v[4], v[5], v[6], v[7]};
    } else if constexpr (PREC == RCH_PREC_BF16) {
        bf8 out;
#pragma unroll
        for (int j = 0; j < 8; ++j) out[j] = static_cast<__bf16>(v[j]);
        gout<bf8>(P.dst_ptr)[q] = out;
    } else {
        const float pre = pow2f(block_exp[b]);
        h8 out;
#pragma unroll
        for (int j = 0; j < 8; ++j) out[j] = static_cast<_Float16>(v[j] * pre);
        gout<h8>(P.dst_ptr)[q] = out;
    }
}

template <int PREC>
__global__ void __launch_bounds__(256) basis_pack_kernel(const rch_pack* __restrict__ packs) {
    // The whole descriptor is read up front (one round of scalar loads): reading fields where they
    // are used chains several dependent memory round trips.
    basis_pack_body<PREC>(packs[blockIdx.z]);
}

// Pack descriptors passed by value (the no-allocation entry point has no device memory of the
// caller's to hold them).
constexpr int kNoAllocMaxPacks = 8;
struct PackArgs {
    rch_pack pack[kNoAllocMaxPacks];
};

template <int PREC>
__global__ void __launch_bounds__(256) basis_pack_args_kernel(const PackArgs args) {
    basis_pack_body<PREC>(args.pack[blockIdx.z]);
}

// ---------------------------------------------------------------------------------------------
// Coefficient bound (float sources, fp16 modes)
// ---------------------------------------------------------------------------------------------

__global__ void __launch_bounds__(256) coefficient_bound_kernel(const rch_job* __restrict__ jobs,
                                                                const int32_t* __restrict__ tiles, int k_tiles,
                                                                int32_t* __restrict__ scratch) {
    const int tile = blockIdx.x / k_tiles, kt = blockIdx.x - tile * k_tiles;
    const rch_job* J = jobs + tiles[2 * tile];
    const int64_t t0 = tiles[2 * tile + 1];
    if (J->bound_index < 0) return;
    const int dtype = static_cast<int>(J->src_dtype);
    float m = 0.0f;
    // 128 tokens x 64 rank columns per block; thread = (token, 32 columns).
    const int64_t t = t0 + (threadIdx.x >> 1);
    const int k0 = kt * 64 + (threadIdx.x & 1) * 32;
    if (t < J->tokens) {
        for (int k = k0; k < k0 + 32 && k < J->rank; ++k)
            m = fmaxf(m, fabsf(load_value(J->src_ptr, t * J->src_row_stride + k * J->src_col_stride, dtype)));
    }
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    __shared__ float partial[4];
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        m = fmaxf(fmaxf(partial[0], partial[1]), fmaxf(partial[2], partial[3]));
        atomicMax(reinterpret_cast<unsigned int*>(scratch + J->bound_index), __float_as_uint(m));  // vector atomic
    }
}

// ---------------------------------------------------------------------------------------------
// Dense rows -> RoPE -> cast -> store
// ---------------------------------------------------------------------------------------------

__global__ void __launch_bounds__(256) rope_store_kernel(const rch_job* __restrict__ jobs,
                                                         const int32_t* __restrict__ tiles, int c_tiles, int channels,
                                                         int head_dim, int out_dtype) {
    const int tile = blockIdx.x / c_tiles, ct = blockIdx.x - tile * c_tiles;
    const rch_job* J = jobs + tiles[2 * tile];
    const int64_t t0 = tiles[2 * tile + 1];
    // 128 tokens x 64 channels per block: thread = (token pair of rows, 16 channels).
    const int c0 = ct * 64 + (threadIdx.x & 3) * 16;
    const int rope = static_cast<int>(J->rope);
    const int dtype = static_cast<int>(J->src_dtype);
    for (int rep = 0; rep < 2; ++rep) {
        const int64_t t = t0 + (threadIdx.x >> 2) + 64 * rep;
        if (t >= J->tokens || c0 >= channels) continue;
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i)
            v[i] = c0 + i < channels ? load_value(J->src_ptr, t * J->src_row_stride + (c0 + i) * J->src_col_stride, dtype) : 0.0f;
        if (rope != RCH_ROPE_NONE) {
            const Coords c = coords(J, static_cast<int>(t));
            apply_rope(J, rope, v, c0, channels, head_dim, t, c.f, c.y, c.x);
        }
        store16(J, v, c0, channels, head_dim, t, out_dtype);
    }
}

// ---------------------------------------------------------------------------------------------
// Staged comparison path: unpack -> library GEMM -> RoPE / cast / store
// ---------------------------------------------------------------------------------------------

// The coefficient prescale exponent of a job in the fp16 modes: the host's, or the one of the
// device bound that rch_coefficient_bound left in its scratch word.
__device__ __forceinline__ int staged_exponent(const rch_job* J, int precision, const int32_t* scratch) {
    if (precision != RCH_PREC_FP16) return 0;
    if (J->bound_index >= 0) return prescale_exponent(__int_as_float(scratch[J->bound_index]));
    return static_cast<int>(J->coef_exp);
}

// One coefficient of token t, rank column k: dequantized with two roundings (uint8 rows,
// pictures) or read as is (float sources), in fp32.
template <int SRC>
__device__ __forceinline__ float staged_coefficient(const rch_job* J, int64_t t, int k, const Coords& c) {
    if constexpr (SRC == RCH_SRC_FLOAT) {
        return load_value(J->src_ptr, t * J->src_row_stride + k * J->src_col_stride, static_cast<int>(J->src_dtype));
    } else {
        const uint32_t q = SRC == RCH_SRC_U8 ? gin<uint8_t>(J->src_ptr)[t * J->src_row_stride + k * J->src_col_stride]
                                             : gin<uint8_t>(J->src_ptr)[picture_offset(J, k, c)];
        return dequant(q, gin<float>(J->scale_ptr)[k], gin<float>(J->offset_ptr)[k]);
    }
}

// Work rows [rows[job] + t] of the dense [rows, rank] coefficient matrix of one GEMM: 128 tokens x
// 64 rank columns per workgroup, thread = (token, 4 consecutive columns), 8 tokens per thread.
// fp16: times 2^e (exact), then one rounding to the work dtype, as the reference's unpack pass
// (reelcache/restore_kernels.py:1518-1554).
template <int SRC, int WORK>
__global__ void __launch_bounds__(256) staged_unpack_kernel(const rch_job* __restrict__ jobs,
                                                            const int32_t* __restrict__ tiles, int k_tiles,
                                                            const int64_t* __restrict__ rows, int64_t work,
                                                            int64_t work_stride, int precision,
                                                            const int32_t* __restrict__ scratch) {
    const int tile = blockIdx.x / k_tiles, kt = blockIdx.x - tile * k_tiles;
    const int job = tiles[2 * tile];
    const rch_job* J = jobs + job;
    const int64_t t0 = tiles[2 * tile + 1];
    const int rank = static_cast<int>(J->rank);
    const int k0 = kt * 64 + (threadIdx.x & 15) * 4;
    if (k0 >= rank) return;
    const float pre = pow2f(staged_exponent(J, precision, scratch));
    const int64_t first = rows[job];
    for (int rep = 0; rep < 8; ++rep) {
        const int64_t t = t0 + (threadIdx.x >> 4) + 16 * rep;
        if (t >= J->tokens) break;
        const Coords c = coords(J, static_cast<int>(t));
        const int64_t at = (first + t) * work_stride;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = k0 + j;
            if (k >= rank) break;
            const float a = __fmul_rn(staged_coefficient<SRC>(J, t, k, c), pre);
            if constexpr (WORK == RCH_DT_F32) gout<float>(work)[at + k] = a;
            else if constexpr (WORK == RCH_DT_F16) gout<_Float16>(work)[at + k] = static_cast<_Float16>(a);
            else gout<__bf16>(work)[at + k] = static_cast<__bf16>(a);
        }
    }
}

// fp32 product rows [rows[job] + t] -> times 2^-e (fp16) -> RoPE -> cast -> native store
// (reelcache/restore_kernels.py:1557-1585 with PRESCALE).
__global__ void __launch_bounds__(256) staged_store_kernel(const rch_job* __restrict__ jobs,
                                                           const int32_t* __restrict__ tiles, int c_tiles,
                                                           const int64_t* __restrict__ rows, int64_t product,
                                                           int64_t product_stride, int channels, int head_dim,
                                                           int out_dtype, int precision,
                                                           const int32_t* __restrict__ scratch) {
    const int tile = blockIdx.x / c_tiles, ct = blockIdx.x - tile * c_tiles;
    const int job = tiles[2 * tile];
    const rch_job* J = jobs + job;
    const int64_t t0 = tiles[2 * tile + 1];
    const int c0 = ct * 64 + (threadIdx.x & 3) * 16;
    const int rope = static_cast<int>(J->rope);
    const float inverse = pow2f(-staged_exponent(J, precision, scratch));
    const int64_t first = rows[job];
    for (int rep = 0; rep < 2; ++rep) {
        const int64_t t = t0 + (threadIdx.x >> 2) + 64 * rep;
        if (t >= J->tokens || c0 >= channels) continue;
        const RCH_GLOBAL float* row = gin<float>(product) + (first + t) * product_stride;
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = c0 + i < channels ? __fmul_rn(row[c0 + i], inverse) : 0.0f;
        if (rope != RCH_ROPE_NONE) {
            const Coords c = coords(J, static_cast<int>(t));
            apply_rope(J, rope, v, c0, channels, head_dim, t, c.f, c.y, c.x);
        }
        store16(J, v, c0, channels, head_dim, t, out_dtype);
    }
}

template <int SRC>
void launch_staged_unpack(int work_dtype, dim3 grid, hipStream_t s, const rch_job* jobs, const int32_t* tiles,
                          int k_tiles, const int64_t* rows, int64_t work, int64_t work_stride, int precision,
                          const int32_t* scratch) {
    switch (work_dtype) {
        case RCH_DT_F32:
            hipLaunchKernelGGL((staged_unpack_kernel<SRC, RCH_DT_F32>), grid, dim3(256), 0, s, jobs, tiles, k_tiles,
                               rows, work, work_stride, precision, scratch);
            break;
        case RCH_DT_F16:
            hipLaunchKernelGGL((staged_unpack_kernel<SRC, RCH_DT_F16>), grid, dim3(256), 0, s, jobs, tiles, k_tiles,
                               rows, work, work_stride, precision, scratch);
            break;
        default:
            hipLaunchKernelGGL((staged_unpack_kernel<SRC, RCH_DT_BF16>), grid, dim3(256), 0, s, jobs, tiles, k_tiles,
                               rows, work, work_stride, precision, scratch);
            break;
    }
}

bool valid_out(int out_dtype) {
    return out_dtype == RCH_DT_F32 || out_dtype == RCH_DT_F16 || out_dtype == RCH_DT_BF16;
}

}  // namespace
}  // namespace rch

using namespace rch;

extern "C" {

int rch_fragment_bytes(int precision) { return precision == RCH_PREC_FP32 ? 32 : 16; }

int rch_basis_pack(const rch_pack* packs_dev, int n_packs, int64_t max_nblocks, int64_t max_ksteps, int precision,
                   void* stream) {
    if (!packs_dev || n_packs <= 0 || n_packs > 65535 || max_nblocks <= 0 || max_nblocks > 0x7fffffff ||
        max_ksteps <= 0 || max_ksteps > 2 * 65535)
        return fail(RCH_E_CONFIG, "rch_basis_pack: invalid arguments");
    const dim3 grid(static_cast<unsigned>((max_nblocks + 1) / 2), static_cast<unsigned>((max_ksteps + 1) / 2), n_packs);
    hipStream_t s = as_stream(stream);
    switch (precision) {
        case RCH_PREC_FP32: hipLaunchKernelGGL(basis_pack_kernel<RCH_PREC_FP32>, grid, dim3(256), 0, s, packs_dev); break;
        case RCH_PREC_FP16: hipLaunchKernelGGL(basis_pack_kernel<RCH_PREC_FP16>, grid, dim3(256), 0, s, packs_dev); break;
        case RCH_PREC_FP16X2: hipLaunchKernelGGL(basis_pack_kernel<RCH_PREC_FP16X2>, grid, dim3(256), 0, s, packs_dev); break;
        case RCH_PREC_BF16: hipLaunchKernelGGL(basis_pack_kernel<RCH_PREC_BF16>, grid, dim3(256), 0, s, packs_dev); break;
        default: return fail(RCH_E_UNSUPPORTED, "precision %d has no matrix-core path on gfx950", precision);
    }
    return check_launch("rch_basis_pack");
}

int rch_coefficient_bound(const rch_job* jobs_dev, int n_jobs, const int32_t* tiles_dev, int n_tiles, int max_rank,
                          int32_t* scratch_dev, void* stream) {
    if (!jobs_dev || !tiles_dev || !scratch_dev || n_jobs <= 0 || n_tiles <= 0 || max_rank <= 0)
        return fail(RCH_E_CONFIG, "rch_coefficient_bound: invalid arguments");
    const int k_tiles = (max_rank + 63) / 64;
    const int64_t blocks = static_cast<int64_t>(n_tiles) * k_tiles;
    if (blocks > 0x7fffffff) return fail(RCH_E_CONFIG, "rch_coefficient_bound: grid too large");
    hipLaunchKernelGGL(coefficient_bound_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, as_stream(stream),
                       jobs_dev, tiles_dev, k_tiles, scratch_dev);
    return check_launch("rch_coefficient_bound");
}

// The kernel an rch_restore launch group runs: the straight-line variant (restore_fast.h) when
// the group qualifies and one is compiled for its rank, else the general restore_kernel.
struct Launch {
    const void* fn;
    bool fast;
    int ks;
    bool chunked;
    int threads;  // workgroup size
    bool stream;  // restore_stream_kernel (RCH_GF_STREAM)
};

static int pick_launch(int precision, int source_kind, int max_ksteps, int head_dim, int out_dtype, int group_flags,
                       Launch* out) {
    if (group_flags & RCH_GF_STREAM) {
        if (!(group_flags & RCH_GF_FAST) || (group_flags & (RCH_GF_HEAD_PAIRS | RCH_GF_SPLIT_RANK)) ||
            precision != RCH_PREC_FP16X2 || source_kind != RCH_SRC_U8 || head_dim != 128)
            return fail(RCH_E_CONFIG, "RCH_GF_STREAM needs RCH_GF_FAST alone, fp16x2, uint8 code rows and head_dim 128");
        int ks = 0;
        const int rope = !(group_flags & RCH_GF_ROPE) ? kRopeNone
                         : ((group_flags & RCH_GF_DENSE_ROPE) ? kRopeDense : kRopeSections);
        StreamFn fn = pick_stream_fp16x2(max_ksteps, rope, out_dtype, &ks);
        if (!fn) return fail(RCH_E_CONFIG, "RCH_GF_STREAM: no stream variant covers %d rank steps", max_ksteps);
        *out = {reinterpret_cast<const void*>(fn), false, ks, false, kThreads, true};
        return RCH_OK;
    }
    if ((group_flags & RCH_GF_FAST) && head_dim % 32 == 0 &&
        (source_kind == RCH_SRC_U8 || source_kind == RCH_SRC_PICTURE)) {
        const bool rope = (group_flags & RCH_GF_ROPE) != 0;
        if ((group_flags & RCH_GF_HEAD_PAIRS) && (group_flags & RCH_GF_SPLIT_RANK))
            return fail(RCH_E_CONFIG, "RCH_GF_HEAD_PAIRS and RCH_GF_SPLIT_RANK exclude each other");
        if ((group_flags & RCH_GF_SPLIT_RANK) && source_kind != RCH_SRC_U8)
            return fail(RCH_E_CONFIG, "RCH_GF_SPLIT_RANK takes uint8 code rows only");
        const int shape = (group_flags & RCH_GF_SPLIT_RANK) ? kRankHalves
                          : ((group_flags & RCH_GF_HEAD_PAIRS) ? kHeadPairs : kOneHead);
        FastFn fn = nullptr;
        int ks = 0;
        switch (precision) {
            case RCH_PREC_FP16: fn = pick_fast_fp16(max_ksteps, rope, out_dtype, shape, &ks); break;
            case RCH_PREC_FP16X2: fn = pick_fast_fp16x2(max_ksteps, rope, out_dtype, shape, &ks); break;
            case RCH_PREC_BF16: fn = pick_fast_bf16(max_ksteps, rope, out_dtype, shape, &ks); break;
            default: break;
        }
        if (fn) {
            *out = {reinterpret_cast<const void*>(fn), true, ks, false, shape == kRankHalves ? 2 * kThreads : kThreads,
                    false};
            return RCH_OK;
        }
    }
    // Head-pair work units and rank halves exist only in the straight-line kernel.
    if (group_flags & (RCH_GF_HEAD_PAIRS | RCH_GF_SPLIT_RANK))
        return fail(RCH_E_CONFIG, "RCH_GF_HEAD_PAIRS / RCH_GF_SPLIT_RANK: no straight-line variant covers %d rank "
                    "steps here", max_ksteps);
    RestoreVariant variant;
    switch (precision) {
        case RCH_PREC_FP32: variant = pick_restore_fp32(source_kind, max_ksteps); break;
        case RCH_PREC_FP16: variant = pick_restore_fp16(source_kind, max_ksteps); break;
        case RCH_PREC_FP16X2: variant = pick_restore_fp16x2(source_kind, max_ksteps); break;
        case RCH_PREC_BF16: variant = pick_restore_bf16(source_kind, max_ksteps); break;
        default: return fail(RCH_E_UNSUPPORTED, "precision %d has no matrix-core path on gfx950", precision);
    }
    if (!variant.fn) return fail(RCH_E_CONFIG, "source kind %d is not a coefficient source", source_kind);
    *out = {reinterpret_cast<const void*>(variant.fn), false, variant.ks, variant.chunked, kThreads, false};
    return RCH_OK;
}

int rch_restore_occupancy(int precision, int source_kind, int max_ksteps, int head_dim, int out_dtype, int group_flags,
                          int* blocks_per_cu) {
    if (!blocks_per_cu || max_ksteps <= 0 || head_dim <= 0)
        return fail(RCH_E_CONFIG, "rch_restore_occupancy: invalid arguments");
    Launch launch;
    const int status = pick_launch(precision, source_kind, max_ksteps, head_dim, out_dtype, group_flags, &launch);
    if (status) return status;
    int blocks = 0;
    const hipError_t error = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, launch.fn, launch.threads, 0);
    if (error != hipSuccess)
        return fail(RCH_E_LAUNCH, "rch_restore_occupancy: %s", hipGetErrorString(error));
    *blocks_per_cu = blocks;
    return RCH_OK;
}

static int check_restore_args(const char* what, const rch_job* jobs_dev, int n_jobs, const int32_t* tiles_dev,
                              int n_tiles, const int32_t* bounds_dev, int grid, int channels, int head_dim,
                              int out_dtype, int max_ksteps, int group_flags) {
    if (!jobs_dev || !tiles_dev || !bounds_dev || n_jobs <= 0 || n_tiles <= 0 || grid <= 0 || channels <= 0 ||
        head_dim <= 0 || head_dim % 2 || max_ksteps <= 0 ||
        static_cast<int64_t>(n_tiles) * ((channels + 31) / 32) > 0x7fffffff)
        return fail(RCH_E_CONFIG, "%s: invalid launch arguments", what);
    if (!valid_out(out_dtype)) return fail(RCH_E_CONFIG, "%s: output dtype must be f32, f16 or bf16", what);
    if ((group_flags & RCH_GF_FAST) && channels % head_dim)
        return fail(RCH_E_CONFIG, "%s: RCH_GF_FAST needs channels == heads * head_dim", what);
    if ((group_flags & RCH_GF_HEAD_PAIRS) && (!(group_flags & RCH_GF_FAST) || (channels / head_dim) % 2))
        return fail(RCH_E_CONFIG, "%s: RCH_GF_HEAD_PAIRS needs RCH_GF_FAST and an even head count", what);
    return RCH_OK;
}

// Launches the kernel pick_launch chose for a group; pack_base is added to every rch_job.pack_ptr.
static void launch_restore(const Launch& launch, const rch_job* jobs_dev, const int32_t* tiles_dev, int n_tiles,
                           const int32_t* bounds_dev, int grid, int channels, int head_dim, int out_dtype,
                           int max_ksteps, const int32_t* scratch_dev, int64_t pack_base, hipStream_t s) {
    if (launch.stream) {
        hipLaunchKernelGGL(reinterpret_cast<StreamFn>(const_cast<void*>(launch.fn)), dim3(static_cast<unsigned>(grid)),
                           dim3(kThreads), 0, s, jobs_dev, tiles_dev, bounds_dev, n_tiles, channels / head_dim,
                           pack_base);
    } else if (launch.fast) {
        hipLaunchKernelGGL(reinterpret_cast<FastFn>(const_cast<void*>(launch.fn)), dim3(static_cast<unsigned>(grid)),
                           dim3(static_cast<unsigned>(launch.threads)), 0, s, jobs_dev, tiles_dev, bounds_dev,
                           scratch_dev, pack_base, channels / head_dim, head_dim);
    } else {
        const int nk = launch.chunked ? (max_ksteps + launch.ks - 1) / launch.ks : 1;
        hipLaunchKernelGGL(reinterpret_cast<RestoreFn>(const_cast<void*>(launch.fn)), dim3(static_cast<unsigned>(grid)),
                           dim3(kThreads), 0, s, jobs_dev, tiles_dev, bounds_dev, scratch_dev, pack_base, nk, channels,
                           head_dim, out_dtype);
    }
}

int rch_restore(const rch_job* jobs_dev, int n_jobs, const int32_t* tiles_dev, int n_tiles, const int32_t* bounds_dev,
                int grid, int channels, int head_dim, int source_kind, int out_dtype, int precision, int max_ksteps,
                int group_flags, const int32_t* scratch_dev, void* stream) {
    if (!scratch_dev) return fail(RCH_E_CONFIG, "rch_restore: invalid launch arguments");
    int status = check_restore_args("rch_restore", jobs_dev, n_jobs, tiles_dev, n_tiles, bounds_dev, grid, channels,
                                    head_dim, out_dtype, max_ksteps, group_flags);
    if (status) return status;
    Launch launch;
    status = pick_launch(precision, source_kind, max_ksteps, head_dim, out_dtype, group_flags, &launch);
    if (status) return status;
    launch_restore(launch, jobs_dev, tiles_dev, n_tiles, bounds_dev, grid, channels, head_dim, out_dtype, max_ksteps,
                   scratch_dev, 0, as_stream(stream));
    return check_launch("rch_restore");
}

// The pair kernel of two head-pair groups, or nullptr when none is compiled for them.
static PairFn pick_pair_launch(int precision, int source_kind, int ksteps0, int ksteps1, int head_dim, int out_dtype,
                               int* chosen0, int* chosen1) {
    *chosen0 = *chosen1 = 0;
    if (head_dim % 32 || ksteps0 <= 0 || ksteps1 <= 0 ||
        (source_kind != RCH_SRC_U8 && source_kind != RCH_SRC_PICTURE))
        return nullptr;
    // fp16x2 only: in the single-product modes the two groups' units cost about the same and one
    // launch per group measured as fast.
    return precision == RCH_PREC_FP16X2 ? pick_pair_fp16x2(ksteps0, ksteps1, out_dtype, chosen0, chosen1) : nullptr;
}

int rch_restore_pair_occupancy(int precision, int source_kind, int ksteps0, int ksteps1, int head_dim, int out_dtype,
                               int* blocks_per_cu) {
    if (!blocks_per_cu) return fail(RCH_E_CONFIG, "rch_restore_pair_occupancy: invalid arguments");
    *blocks_per_cu = 0;
    int chosen0 = 0, chosen1 = 0;
    const PairFn fn = pick_pair_launch(precision, source_kind, ksteps0, ksteps1, head_dim, out_dtype, &chosen0,
                                       &chosen1);
    if (!fn) return RCH_OK;  // no pair kernel: the groups launch one by one
    int blocks = 0;
    const hipError_t error = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, kThreads, 0);
    if (error != hipSuccess)
        return fail(RCH_E_LAUNCH, "rch_restore_pair_occupancy: %s", hipGetErrorString(error));
    *blocks_per_cu = blocks;
    return RCH_OK;
}

int rch_restore_pair(const rch_job* jobs_dev, int n_jobs, const int32_t* tiles_dev, int n_tiles0, int n_tiles1,
                     const int32_t* bounds_dev, int grid, int channels, int head_dim, int source_kind, int out_dtype,
                     int precision, int ksteps0, int ksteps1, const int32_t* scratch_dev, void* stream) {
    if (!scratch_dev || n_tiles0 <= 0 || n_tiles1 <= 0 || n_tiles0 > 0x7fffffff - n_tiles1)
        return fail(RCH_E_CONFIG, "rch_restore_pair: invalid launch arguments");
    const int flags = RCH_GF_FAST | RCH_GF_HEAD_PAIRS;
    int status = check_restore_args("rch_restore_pair", jobs_dev, n_jobs, tiles_dev, n_tiles0 + n_tiles1, bounds_dev,
                                    grid, channels, head_dim, out_dtype, ksteps0 > ksteps1 ? ksteps0 : ksteps1, flags);
    if (status) return status;
    int chosen0 = 0, chosen1 = 0;
    const PairFn fn = pick_pair_launch(precision, source_kind, ksteps0, ksteps1, head_dim, out_dtype, &chosen0,
                                       &chosen1);
    if (!fn)
        return fail(RCH_E_CONFIG, "rch_restore_pair: no pair kernel covers precision %d, output dtype %d, %d and %d "
                    "rank steps", precision, out_dtype, ksteps0, ksteps1);
    // Units of the first group: its tiles x head-pair units per tile (checked above to fit int32).
    const int heads = channels / head_dim;
    const int split_unit = n_tiles0 * ((heads / 2) * (head_dim / 32));
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, as_stream(stream), jobs_dev,
                       tiles_dev, bounds_dev, scratch_dev, int64_t(0), heads, head_dim, split_unit);
    return check_launch("rch_restore_pair");
}

int rch_rope_store(const rch_job* jobs_dev, int n_jobs, const int32_t* tiles_dev, int n_tiles, int channels,
                   int head_dim, int out_dtype, void* stream) {
    if (!jobs_dev || !tiles_dev || n_jobs <= 0 || n_tiles <= 0 || channels <= 0 || head_dim <= 0 || head_dim % 2)
        return fail(RCH_E_CONFIG, "rch_rope_store: invalid launch arguments");
    if (!valid_out(out_dtype)) return fail(RCH_E_CONFIG, "rch_rope_store: output dtype must be f32, f16 or bf16");
    const int c_tiles = (channels + 63) / 64;
    const int64_t blocks = static_cast<int64_t>(n_tiles) * c_tiles;
    if (blocks > 0x7fffffff) return fail(RCH_E_CONFIG, "rch_rope_store: grid too large");
    hipLaunchKernelGGL(rope_store_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, as_stream(stream),
                       jobs_dev, tiles_dev, c_tiles, channels, head_dim, out_dtype);
    return check_launch("rch_rope_store");
}

int rch_staged_unpack(const rch_job* jobs_dev, int n_jobs, const int32_t* tiles_dev, int n_tiles,
                      const int64_t* rows_dev, void* work, int64_t work_stride, int max_rank, int source_kind,
                      int work_dtype, int precision, const int32_t* scratch_dev, void* stream) {
    if (!jobs_dev || !tiles_dev || !rows_dev || !work || !scratch_dev || n_jobs <= 0 || n_tiles <= 0 ||
        max_rank <= 0 || work_stride < max_rank)
        return fail(RCH_E_CONFIG, "rch_staged_unpack: invalid launch arguments");
    if (work_dtype != RCH_DT_F32 && work_dtype != RCH_DT_F16 && work_dtype != RCH_DT_BF16)
        return fail(RCH_E_CONFIG, "rch_staged_unpack: work dtype must be f32, f16 or bf16");
    if (precision != RCH_PREC_FP32 && precision != RCH_PREC_FP16 && precision != RCH_PREC_BF16)
        return fail(RCH_E_UNSUPPORTED, "rch_staged_unpack: the staged path runs fp32, fp16 or bf16 (precision %d)",
                    precision);
    const int k_tiles = (max_rank + 63) / 64;
    const int64_t blocks = static_cast<int64_t>(n_tiles) * k_tiles;
    if (blocks > 0x7fffffff) return fail(RCH_E_CONFIG, "rch_staged_unpack: grid too large");
    const dim3 grid(static_cast<unsigned>(blocks));
    const int64_t address = reinterpret_cast<int64_t>(work);
    hipStream_t s = as_stream(stream);
    switch (source_kind) {
        case RCH_SRC_FLOAT:
            launch_staged_unpack<RCH_SRC_FLOAT>(work_dtype, grid, s, jobs_dev, tiles_dev, k_tiles, rows_dev, address,
                                                work_stride, precision, scratch_dev);
            break;
        case RCH_SRC_U8:
            launch_staged_unpack<RCH_SRC_U8>(work_dtype, grid, s, jobs_dev, tiles_dev, k_tiles, rows_dev, address,
                                             work_stride, precision, scratch_dev);
            break;
        case RCH_SRC_PICTURE:
            launch_staged_unpack<RCH_SRC_PICTURE>(work_dtype, grid, s, jobs_dev, tiles_dev, k_tiles, rows_dev, address,
                                                  work_stride, precision, scratch_dev);
            break;
        default: return fail(RCH_E_CONFIG, "rch_staged_unpack: source kind %d is not a coefficient source", source_kind);
    }
    return check_launch("rch_staged_unpack");
}

int rch_staged_store(const rch_job* jobs_dev, int n_jobs, const int32_t* tiles_dev, int n_tiles,
                     const int64_t* rows_dev, const void* product, int64_t product_stride, int channels, int head_dim,
                     int out_dtype, int precision, const int32_t* scratch_dev, void* stream) {
    if (!jobs_dev || !tiles_dev || !rows_dev || !product || !scratch_dev || n_jobs <= 0 || n_tiles <= 0 ||
        channels <= 0 || head_dim <= 0 || head_dim % 2 || product_stride < channels)
        return fail(RCH_E_CONFIG, "rch_staged_store: invalid launch arguments");
    if (!valid_out(out_dtype)) return fail(RCH_E_CONFIG, "rch_staged_store: output dtype must be f32, f16 or bf16");
    if (precision != RCH_PREC_FP32 && precision != RCH_PREC_FP16 && precision != RCH_PREC_BF16)
        return fail(RCH_E_UNSUPPORTED, "rch_staged_store: the staged path runs fp32, fp16 or bf16 (precision %d)",
                    precision);
    const int c_tiles = (channels + 63) / 64;
    const int64_t blocks = static_cast<int64_t>(n_tiles) * c_tiles;
    if (blocks > 0x7fffffff) return fail(RCH_E_CONFIG, "rch_staged_store: grid too large");
    hipLaunchKernelGGL(staged_store_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, as_stream(stream),
                       jobs_dev, tiles_dev, c_tiles, rows_dev, reinterpret_cast<int64_t>(product), product_stride,
                       channels, head_dim, out_dtype, precision, scratch_dev);
    return check_launch("rch_staged_store");
}

}  // extern "C"

// ---------------------------------------------------------------------------------------------
// Restore without allocation (rch_restore_noalloc): the packed bases and their block exponents
// live in this file's static device array instead of memory the caller allocates.
// ---------------------------------------------------------------------------------------------

// Bytes [0, RCH_NOALLOC_WORD_BYTES): int32 block exponents; the packed fragments follow.  Each GPU
// the library runs on holds its own copy until the process ends.
static __device__ __align__(256) uint8_t scratch[RCH_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex scratch_lock;
void* scratch_ptr[kMaxDevices];  // device address of `scratch` per device, set on its first call

// The current device's address of `scratch`.  In host code the array's name is only a stand-in:
// every kernel argument and address computed here uses this pointer.
int current_scratch(void** out) {
    int device = -1;
    hipError_t error = hipGetDevice(&device);
    if (error != hipSuccess) return fail(RCH_E_LAUNCH, "rch_restore_noalloc: hipGetDevice: %s", hipGetErrorString(error));
    if (device < 0 || device >= kMaxDevices) return fail(RCH_E_UNSUPPORTED, "rch_restore_noalloc: device %d", device);
    std::lock_guard<std::mutex> hold(scratch_lock);
    if (!scratch_ptr[device]) {
        void* ptr = nullptr;
        error = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (error != hipSuccess || !ptr)
            return fail(RCH_E_LAUNCH, "rch_restore_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(error));
        scratch_ptr[device] = ptr;
    }
    *out = scratch_ptr[device];
    return RCH_OK;
}

}  // namespace

extern "C" {

int rch_restore_noalloc(const rch_pack* packs_host, int n_packs, const rch_job* jobs_dev, int n_jobs,
                        const int32_t* tiles_dev, int n_tiles, const int32_t* bounds_dev, int grid, int channels,
                        int head_dim, int source_kind, int out_dtype, int precision, int max_ksteps, int group_flags,
                        void* stream) {
    if (!packs_host || n_packs <= 0)
        return fail(RCH_E_CONFIG, "rch_restore_noalloc: invalid pack descriptors");
    if (n_packs > kNoAllocMaxPacks)
        return fail(RCH_E_CONFIG, "rch_restore_noalloc: %d bases in one call, at most %d", n_packs, kNoAllocMaxPacks);
    int status = check_restore_args("rch_restore_noalloc", jobs_dev, n_jobs, tiles_dev, n_tiles, bounds_dev, grid,
                                    channels, head_dim, out_dtype, max_ksteps, group_flags);
    if (status) return status;
    if (precision != RCH_PREC_FP32 && precision != RCH_PREC_FP16 && precision != RCH_PREC_FP16X2 &&
        precision != RCH_PREC_BF16)
        return fail(RCH_E_UNSUPPORTED, "precision %d has no matrix-core path on gfx950", precision);
    // The layout: pack i's exponents at word E_i = sum_{j<i} nblocks_j, its fragments at byte
    // F_i = sum_{j<i} round_up(ksteps_j * nblocks_j * 64 * fragment bytes, 256) of the fragment region.
    const int64_t fragment = rch_fragment_bytes(precision);
    int64_t words = 0, bytes = 0, max_nblocks = 0, max_pack_steps = 0;
    // The kernel first: a stream variant reads slabs of exactly its own ks rank steps.
    Launch launch;
    status = pick_launch(precision, source_kind, max_ksteps, head_dim, out_dtype, group_flags, &launch);
    if (status) return status;
    PackArgs args;
    void* base = nullptr;
    status = current_scratch(&base);
    if (status) return status;
    const int64_t word_base = reinterpret_cast<int64_t>(base);
    const int64_t fragment_base = word_base + RCH_NOALLOC_WORD_BYTES;
    for (int i = 0; i < n_packs; ++i) {
        const rch_pack& P = packs_host[i];
        const bool slabs = P.kind == RCH_PACK_STREAM;
        if (P.rank <= 0 || P.channels <= 0 || (P.kind != RCH_PACK_FRAGMENTS && !slabs) || slabs != launch.stream ||
            (slabs ? (!stream_pack_steps(P.ksteps) || P.ksteps != launch.ks || P.ksteps < (P.rank + 15) / 16 ||
                      P.nblocks != P.channels / 32 || P.channels % 128)
                   : (P.ksteps != (P.rank + 15) / 16 || P.nblocks != 2 * ((P.channels + 63) / 64))))
            return fail(RCH_E_CONFIG, "rch_restore_noalloc: pack %d: kind / ksteps / nblocks do not match its rank / "
                        "channels or the launch group's kernel (stream slabs: ksteps 4, 8, 12 or 16, the variant's)",
                        i);
        args.pack[i] = P;
        args.pack[i].exp_ptr = word_base + 4 * words;
        args.pack[i].dst_ptr = fragment_base + bytes;
        words += slabs ? 0 : P.nblocks;
        bytes += slabs ? P.nblocks * stream_slab_bytes(P.ksteps)
                       : (P.ksteps * P.nblocks * 64 * fragment + 255) / 256 * 256;
        max_nblocks = P.nblocks > max_nblocks ? P.nblocks : max_nblocks;
        max_pack_steps = P.ksteps > max_pack_steps ? P.ksteps : max_pack_steps;
    }
    if (4 * words > RCH_NOALLOC_WORD_BYTES || bytes > RCH_NOALLOC_SCRATCH_BYTES - RCH_NOALLOC_WORD_BYTES)
        return fail(RCH_E_CONFIG,
                    "rch_restore_noalloc: the packed bases need %lld fragment bytes and %lld exponent words; the "
                    "static scratch holds %d and %d",
                    static_cast<long long>(bytes), static_cast<long long>(words),
                    RCH_NOALLOC_SCRATCH_BYTES - RCH_NOALLOC_WORD_BYTES, RCH_NOALLOC_WORD_BYTES / 4);
    hipStream_t s = as_stream(stream);
    const dim3 pack_grid(static_cast<unsigned>((max_nblocks + 1) / 2), static_cast<unsigned>((max_pack_steps + 1) / 2),
                         static_cast<unsigned>(n_packs));
    switch (precision) {
        case RCH_PREC_FP32: hipLaunchKernelGGL(basis_pack_args_kernel<RCH_PREC_FP32>, pack_grid, dim3(256), 0, s, args); break;
        case RCH_PREC_FP16: hipLaunchKernelGGL(basis_pack_args_kernel<RCH_PREC_FP16>, pack_grid, dim3(256), 0, s, args); break;
        case RCH_PREC_FP16X2: hipLaunchKernelGGL(basis_pack_args_kernel<RCH_PREC_FP16X2>, pack_grid, dim3(256), 0, s, args); break;
        default: hipLaunchKernelGGL(basis_pack_args_kernel<RCH_PREC_BF16>, pack_grid, dim3(256), 0, s, args); break;
    }
    status = check_launch("rch_restore_noalloc (basis pack)");
    if (status) return status;
    launch_restore(launch, jobs_dev, tiles_dev, n_tiles, bounds_dev, grid, channels, head_dim, out_dtype, max_ksteps,
                   reinterpret_cast<const int32_t*>(base), fragment_base, s);
    return check_launch("rch_restore_noalloc");
}

}  // extern "C"
