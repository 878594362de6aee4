#pragma once
// Device code of the fused restore kernel for MI355X (gfx950): dequantize -> MFMA
// rank-view product -> RoPE -> native store.  Included by one translation unit per
// precision (restore_<precision>.hip) so the variants compile in parallel.
//
// Reference: reelcache/restore_kernels.py (_fused_restore_kernel :1447-1515,
// _load_coefficients :1331-1379, _epilogue :1401-1444, _rope_store_kernel
// :1557-1585, _bound_kernel :1588-1606).  The arithmetic contract is the
// reference's: dequantization is float(q) * scale + offset with two roundings,
// fp16 operands are prescaled by an exact power of two, products accumulate in
// fp32, RoPE rotates interleaved pairs in fp32 with fp32 tables, one final cast.
//
// Work decomposition (MI355X-first, not the reference's tiling):
//   * A tile is 128 tokens of one job; a workgroup (4 waves, one 32-token block each)
//     walks a contiguous range of (tile, 32-channel block) units (persistent grid).
//   * The product is computed transposed, out^T[c, t] = Q^T[c, k] * P^T[k, t], with
//     v_mfma_f32_32x32x16_{f16,bf16} (or 32x32x2_f32): channels sit on the MFMA row
//     axis, so each lane's accumulator holds 16 consecutive channels of one token
//     (the basis packer permutes rows to make them consecutive).  RoPE pairs stay
//     inside a lane and each lane writes 32-64 contiguous bytes.
//   * When a workgroup enters a tile, the tile's 8-bit codes and affine are staged
//     into LDS with coalesced loads (pictures are gathered there), and each wave
//     converts its 32 tokens into coefficient fragments (dequantized, prescaled,
//     split hi/lo) held in registers for the rest of the tile.
//   * Basis fragments (one 32-channel block x the rank) are staged in LDS, double
//     buffered, and shared by the 4 waves.
#include "common.h"

namespace rch {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kTileTokens = 32 * kWaves;

// Channel held by MFMA row m of a 32-channel block.  Lane half h of a 32x32 accumulator
// holds rows {8g + 4h + r}; mapping them to 16h + 4g + r puts 16 consecutive channels,
// in accumulator order, in each lane.
__device__ __forceinline__ int block_channel(int m) { return 16 * ((m >> 2) & 1) + 4 * (m >> 3) + (m & 3); }

// Rank index (within a 16-wide step) held by lane half h, element j of an MFMA operand.
// Any bijection works as long as the basis and coefficient fragments agree.
template <int PREC>
__device__ __forceinline__ int k_slot(int h, int j) {
    return PREC == RCH_PREC_FP32 ? 2 * j + h : 8 * h + j;
}

template <int PREC> struct CoefFrag;
template <> struct CoefFrag<RCH_PREC_FP16> { h8 hi; };
template <> struct CoefFrag<RCH_PREC_FP16X2> { h8 hi, lo; };
template <> struct CoefFrag<RCH_PREC_BF16> { bf8 hi; };
template <> struct CoefFrag<RCH_PREC_FP32> { float v[8]; };

// Each fragment is assembled in a fresh vector and assigned whole, so the previous fragment
// is dead while the next is built (element-wise updates would keep it live).
__device__ __forceinline__ void set_frag(CoefFrag<RCH_PREC_FP16>& f, const float (&a)[8], float pre) {
    h8 hi;
#pragma unroll
    for (int j = 0; j < 8; ++j) hi[j] = static_cast<_Float16>(a[j] * pre);
    f.hi = hi;
}
__device__ __forceinline__ void set_frag(CoefFrag<RCH_PREC_FP16X2>& f, const float (&a)[8], float pre) {
    h8 hi, lo;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float v = a[j] * pre;  // exact: power-of-two scale
        const _Float16 head = static_cast<_Float16>(v);
        hi[j] = head;
        lo[j] = static_cast<_Float16>(v - static_cast<float>(head));
    }
    f.hi = hi;
    f.lo = lo;
}
__device__ __forceinline__ void set_frag(CoefFrag<RCH_PREC_BF16>& f, const float (&a)[8], float) {
    bf8 hi;
#pragma unroll
    for (int j = 0; j < 8; ++j) hi[j] = static_cast<__bf16>(a[j]);
    f.hi = hi;
}
__device__ __forceinline__ void set_frag(CoefFrag<RCH_PREC_FP32>& f, const float (&a)[8], float) {
#pragma unroll
    for (int j = 0; j < 8; ++j) f.v[j] = a[j];
}

// Fragments of 8 values that already carry the power-of-two prescale (quantized sources fold it
// into the staged affine: fl(fl(q * s * 2^e) + o * 2^e) = 2^e * fl(fl(q * s) + o) exactly while the
// values stay normal).  Same bits as set_frag(f, a / 2^e, 2^e); conversions run two values at a
// time (v_cvt_pk_f16_f32 rounds to nearest even like the scalar conversion).
__device__ __forceinline__ void set_frag_scaled(CoefFrag<RCH_PREC_FP16>& f, const float (&a)[8]) {
    h8 hi;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const h2 head = __builtin_convertvector((f2{a[2 * p], a[2 * p + 1]}), h2);
        hi[2 * p] = head[0];
        hi[2 * p + 1] = head[1];
    }
    f.hi = hi;
}
__device__ __forceinline__ void set_frag_scaled(CoefFrag<RCH_PREC_FP16X2>& f, const float (&a)[8]) {
    h8 hi, lo;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const f2 v = {a[2 * p], a[2 * p + 1]};
        const h2 head = __builtin_convertvector(v, h2);
        const h2 tail = __builtin_convertvector(v - __builtin_convertvector(head, f2), h2);  // v - hi is exact
        hi[2 * p] = head[0];
        hi[2 * p + 1] = head[1];
        lo[2 * p] = tail[0];
        lo[2 * p + 1] = tail[1];
    }
    f.hi = hi;
    f.lo = lo;
}
__device__ __forceinline__ void set_frag_scaled(CoefFrag<RCH_PREC_BF16>& f, const float (&a)[8]) { set_frag(f, a, 1.0f); }
__device__ __forceinline__ void set_frag_scaled(CoefFrag<RCH_PREC_FP32>& f, const float (&a)[8]) { set_frag(f, a, 1.0f); }

__device__ __forceinline__ float load_value(int64_t base, int64_t index, int dtype) {
    if (dtype == RCH_DT_F32) return gin<float>(base)[index];
    if (dtype == RCH_DT_F16) return static_cast<float>(gin<_Float16>(base)[index]);
    if (dtype == RCH_DT_BF16) return static_cast<float>(gin<__bf16>(base)[index]);
    return static_cast<float>(gin<uint8_t>(base)[index]);
}

// float(q) * scale + offset with two roundings (reelcache/restore_kernels.py:1034-1038).
__device__ __forceinline__ float dequant(uint32_t q, float scale, float offset) {
    return __fadd_rn(__fmul_rn(static_cast<float>(q), scale), offset);
}

template <int PREC>
__device__ __forceinline__ f16v mfma_step(const u4* frag, const CoefFrag<PREC>& c, f16v acc) {
    if constexpr (PREC == RCH_PREC_FP16 || PREC == RCH_PREC_FP16X2) {
        const h8 a = *reinterpret_cast<const h8*>(frag);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, c.hi, acc, 0, 0, 0);
        if constexpr (PREC == RCH_PREC_FP16X2) acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, c.lo, acc, 0, 0, 0);
    } else if constexpr (PREC == RCH_PREC_BF16) {
        const bf8 a = *reinterpret_cast<const bf8*>(frag);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, c.hi, acc, 0, 0, 0);
    } else {
        const f4 a0 = *reinterpret_cast<const f4*>(frag);
        const f4 a1 = *reinterpret_cast<const f4*>(frag + 1);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[j], c.v[j], acc, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[j], c.v[j + 4], acc, 0, 0, 0);
    }
    return acc;
}

// One 16-rank step from a basis fragment already in registers (16-bit modes).
template <int PREC>
__device__ __forceinline__ f16v mfma_frag(u4 frag, const CoefFrag<PREC>& c, f16v acc) {
    static_assert(PREC != RCH_PREC_FP32, "fp32 fragments are 32 bytes");
    if constexpr (PREC == RCH_PREC_BF16) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf8, frag), c.hi, acc, 0, 0, 0);
    } else {
        const h8 a = __builtin_bit_cast(h8, frag);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, c.hi, acc, 0, 0, 0);
        if constexpr (PREC == RCH_PREC_FP16X2) acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, c.lo, acc, 0, 0, 0);
        return acc;
    }
}

// RoPE table row of pair j for a token (separable sections or dense rows).
__device__ __forceinline__ int64_t rope_row(const rch_job* J, int kind, int j, int64_t t, int f, int y, int x) {
    if (kind == RCH_ROPE_DENSE) return J->row_t + t;
    if (j < J->sec_t) return J->row_t + f;
    if (j < J->sec_t + J->sec_h) return J->row_h + y;
    return J->row_w + x;
}

// out_e = e*cos - o*sin, out_o = e*sin + o*cos, each product and sum rounded (no FMA),
// as the reference epilogue compiles with enable_fp_fusion=False (restore_kernels.py:1427, :1998).
__device__ __forceinline__ void rotate(float& e, float& o, float c, float s) {
    const float re = __fsub_rn(__fmul_rn(e, c), __fmul_rn(o, s));
    const float ro = __fadd_rn(__fmul_rn(e, s), __fmul_rn(o, c));
    e = re;
    o = ro;
}

// Rotates v[0..15] (channels c0 .. c0 + 15) of token t.
__device__ __forceinline__ void apply_rope(const rch_job* J, int kind, float (&v)[16], int c0, int channels, int head_dim,
                                           int64_t t, int f, int y, int x) {
    const RCH_GLOBAL float* cos_t = gin<float>(J->cos_ptr);
    const RCH_GLOBAL float* sin_t = gin<float>(J->sin_ptr);
    const int64_t rs = J->rope_row_stride;
    const int d0 = c0 % head_dim;
    if ((J->flags & RCH_JF_ROPE_VEC) && d0 + 16 <= head_dim) {
        const int j0 = d0 >> 1;
        // The 8 pairs share one table row when they lie in one section (always, for dense tables).
        const int64_t s0 = J->sec_t, s1 = J->sec_t + J->sec_h;
        const int first = j0 < s0 ? 0 : (j0 < s1 ? 1 : 2);
        const int last = j0 + 7 < s0 ? 0 : (j0 + 7 < s1 ? 1 : 2);
        if (kind == RCH_ROPE_DENSE || first == last) {
            const int64_t r0 = rope_row(J, kind, j0, t, f, y, x);
            const RCH_GLOBAL f4* cv = reinterpret_cast<const RCH_GLOBAL f4*>(cos_t + r0 * rs + j0);
            const RCH_GLOBAL f4* sv = reinterpret_cast<const RCH_GLOBAL f4*>(sin_t + r0 * rs + j0);
            const f4 ca = cv[0], cb = cv[1], sa = sv[0], sb = sv[1];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                rotate(v[2 * p], v[2 * p + 1], ca[p], sa[p]);
                rotate(v[8 + 2 * p], v[8 + 2 * p + 1], cb[p], sb[p]);
            }
            return;
        }
    }
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const int c = c0 + 2 * p;
        if (c < channels) {
            const int j = (c % head_dim) >> 1;
            const int64_t r = rope_row(J, kind, j, t, f, y, x);
            rotate(v[2 * p], v[2 * p + 1], cos_t[r * rs + j], sin_t[r * rs + j]);
        }
    }
}

// Stores v[0..15] (channels c0 .. c0 + 15 of token t) into the native destination.
__device__ __forceinline__ void store16(const rch_job* J, const float (&v)[16], int c0, int channels, int head_dim,
                                        int64_t t, int out_dtype) {
    const int64_t ts = J->dst_token_stride, hs = J->dst_head_stride, ds = J->dst_dim_stride;
    const int d0 = c0 % head_dim;
    if ((J->flags & RCH_JF_DST_VEC) && c0 + 16 <= channels && d0 + 16 <= head_dim) {
        const int64_t e = t * ts + static_cast<int64_t>(c0 / head_dim) * hs + d0;
        if (out_dtype == RCH_DT_BF16) {
            bf8 lo, hi;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                lo[i] = static_cast<__bf16>(v[i]);
                hi[i] = static_cast<__bf16>(v[i + 8]);
            }
            RCH_GLOBAL bf8* p = gout<bf8>(J->dst_ptr + 2 * e);
            p[0] = lo;
            p[1] = hi;
        } else if (out_dtype == RCH_DT_F16) {
            h8 lo, hi;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                lo[i] = static_cast<_Float16>(v[i]);
                hi[i] = static_cast<_Float16>(v[i + 8]);
            }
            RCH_GLOBAL h8* p = gout<h8>(J->dst_ptr + 2 * e);
            p[0] = lo;
            p[1] = hi;
        } else {
            RCH_GLOBAL f4* p = gout<f4>(J->dst_ptr + 4 * e);
#pragma unroll
            for (int q = 0; q < 4; ++q) p[q] = f4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int c = c0 + i;
        if (c < channels) {
            const int64_t e = t * ts + static_cast<int64_t>(c / head_dim) * hs + static_cast<int64_t>(c % head_dim) * ds;
            if (out_dtype == RCH_DT_BF16) gout<__bf16>(J->dst_ptr)[e] = static_cast<__bf16>(v[i]);
            else if (out_dtype == RCH_DT_F16) gout<_Float16>(J->dst_ptr)[e] = static_cast<_Float16>(v[i]);
            else gout<float>(J->dst_ptr)[e] = v[i];
        }
    }
}

// (frame, row, column) of token t in a job's grid.
struct Coords {
    int f, y, x;
};
__device__ __forceinline__ Coords coords(const rch_job* J, int t) {
    const int plane = static_cast<int>(J->grid_h * J->grid_w);
    const int w = static_cast<int>(J->grid_w);
    Coords c;
    c.f = t / plane;
    const int rest = t - c.f * plane;
    c.y = rest / w;
    c.x = rest - c.y * w;
    return c;
}

// Byte offset (from the picture base) of rank column k of a token in the channel_tiles.v1
// layout (reelcache/restore_kernels.py:23-30, :1340-1364): column k lives in segment
// k // slots; cell i = k % slots uses plane i % planes and grid cell divmod(i // planes, cols).
__device__ __forceinline__ int64_t picture_offset(const rch_job* J, int k, const Coords& c) {
    const int slots = static_cast<int>(J->pic_slots), planes = static_cast<int>(J->pic_planes);
    const int segment = k / slots;
    const int cell = k - segment * slots;
    const int plane = cell % planes;
    const int index = cell / planes;
    const int cols = static_cast<int>(J->pic_grid_cols);
    const int cell_row = index / cols;
    const int cell_col = index - cell_row * cols;
    return gin<int64_t>(J->pic_table_ptr)[static_cast<int64_t>(segment) * J->frames + c.f] + plane * J->pic_plane_stride +
           (static_cast<int64_t>(cell_row) * J->grid_h + c.y) * J->pic_row_stride + cell_col * J->grid_w + c.x;
}

// Loads the cos/sin of the 8 pairs of channels c0 .. c0 + 15 (token t) into registers; the
// values are consumed by rotate16 after the step's products, so the loads overlap the MFMAs.
struct RopeRegs {
    f4 c0, c1, s0, s1;
    bool vec;
};
__device__ __forceinline__ RopeRegs load_rope(const rch_job* J, int kind, int c0, int head_dim, int64_t t, int f,
                                              int y, int x) {
    RopeRegs r;
    r.vec = false;
    const int d0 = c0 % head_dim;
    if ((J->flags & RCH_JF_ROPE_VEC) && d0 + 16 <= head_dim) {
        const int j0 = d0 >> 1;
        const int64_t s0 = J->sec_t, s1 = J->sec_t + J->sec_h;
        const int first = j0 < s0 ? 0 : (j0 < s1 ? 1 : 2);
        const int last = j0 + 7 < s0 ? 0 : (j0 + 7 < s1 ? 1 : 2);
        if (kind == RCH_ROPE_DENSE || first == last) {
            const int64_t row = rope_row(J, kind, j0, t, f, y, x);
            const RCH_GLOBAL f4* cv = reinterpret_cast<const RCH_GLOBAL f4*>(gin<float>(J->cos_ptr) + row * J->rope_row_stride + j0);
            const RCH_GLOBAL f4* sv = reinterpret_cast<const RCH_GLOBAL f4*>(gin<float>(J->sin_ptr) + row * J->rope_row_stride + j0);
            r.c0 = cv[0];
            r.c1 = cv[1];
            r.s0 = sv[0];
            r.s1 = sv[1];
            r.vec = true;
        }
    }
    return r;
}

// Persistent fused restore.  Work units are (tile, 32-channel block) pairs, tile-major;
// workgroup w processes the contiguous unit range [bounds[w'], bounds[w' + 1]) where w'
// is its XCD-swizzled index, so neighbouring ranges share an XCD's L2.  The host sizes
// the grid to the resident capacity, balances the ranges by rank (cost) and launches
// jobs of one rank class (KS) together, so the product loop is a fixed KS steps (steps
// beyond a job's rank read zero fragments).
//
// CHUNKED: the rank exceeds KS steps; each unit runs nk = ceil(max steps / KS) k chunks
// and rebuilds the coefficient fragments per chunk (slower; ranks beyond the register
// budget only).  Otherwise fragments are rebuilt only when the tile changes.
template <int PREC, int SRC, int KS, bool CHUNKED>
__global__ void __launch_bounds__(kThreads, 2)
restore_kernel(const rch_job* __restrict__ jobs, const int32_t* __restrict__ tiles,
               const int32_t* __restrict__ bounds, const int32_t* __restrict__ scratch, int64_t pack_base, int nk,
               int channels, int head_dim, int out_dtype) {
    constexpr int kFrag = PREC == RCH_PREC_FP32 ? 2 : 1;  // u4 per lane fragment
    constexpr int kStepFrags = 64 * kFrag;               // one 16-rank step of one 32-channel block
    constexpr int kBuffer = KS * kStepFrags;
    constexpr int kPerThread = (kBuffer + kThreads - 1) / kThreads;
    constexpr int kRanks = KS * 16;                      // rank columns converted per build
    constexpr int kPitch = kRanks + 8;                   // staged bytes per token (padding spreads LDS banks)
    constexpr bool kStaged = SRC != RCH_SRC_FLOAT;
    constexpr bool kFp16 = PREC == RCH_PREC_FP16 || PREC == RCH_PREC_FP16X2;
    __shared__ u4 lds[2][kBuffer];
    __shared__ __attribute__((aligned(16))) uint8_t codes[kStaged ? kTileTokens * kPitch : 16];
    __shared__ __attribute__((aligned(16))) float affine[kStaged ? 2 * kRanks : 4];

    const int range = xcd_unit(blockIdx.x, gridDim.x);
    const int first_unit = bounds[range];
    const int steps = (bounds[range + 1] - first_unit) * (CHUNKED ? nk : 1);
    if (steps <= 0) return;
    const int blocks_per_tile = (channels + 31) >> 5;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, h = lane >> 5, col = lane & 31;

    // Step st -> (unit, k chunk) -> (tile, channel block).
    auto locate = [&](int st, int& tile, int& block, int& kc) {
        const int unit = first_unit + (CHUNKED ? st / nk : st);
        kc = CHUNKED ? st - (st / nk) * nk : 0;
        tile = unit / blocks_per_tile;
        block = unit - tile * blocks_per_tile;
    };
    // Rank steps of (a job in) this k chunk, clamped to [0, KS].
    auto chunk_steps = [&](const rch_job* job, int kc) {
        return max(0, min(KS, static_cast<int>((job->rank + 15) >> 4) - kc * KS));
    };

    u4 staged[kPerThread];
    auto fetch = [&](int st) {
        int tile, block, kc;
        locate(st, tile, block, kc);
        const rch_job* job = jobs + tiles[2 * tile];
        const int count = chunk_steps(job, kc) * kStepFrags;
        const RCH_GLOBAL u4* pack = gin<u4>(pack_base + job->pack_ptr);
        const int64_t nblocks = job->pack_nblocks;
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int q = tid + i * kThreads;
            if (q < count) {
                const int s = q / kStepFrags, li = q - s * kStepFrags;
                staged[i] = pack[(static_cast<int64_t>(kc * KS + s) * nblocks + block) * kStepFrags + li];
            }
        }
    };
    // Steps beyond the job's rank are written as zeros, so the product loop always runs KS steps.
    auto commit = [&](int st, int buffer) {
        int tile, block, kc;
        locate(st, tile, block, kc);
        const int count = chunk_steps(jobs + tiles[2 * tile], kc) * kStepFrags;
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int q = tid + i * kThreads;
            if (q < kBuffer) lds[buffer][q] = q < count ? staged[i] : u4{0u, 0u, 0u, 0u};
        }
    };

    // Per-lane state of the current tile.
    int current = -1;
    int64_t t = 0;
    bool valid = false;
    Coords xy = {0, 0, 0};
    float pre = 1.0f;
    int coef_exp = 0;

    // Stages the codes of rank columns [kc*kRanks, (kc+1)*kRanks) of the tile's 128 tokens
    // (zero beyond the rank or the job) and their affine into LDS.
    auto stage = [&](const rch_job* J, int t0, int kc) {
        const int k_lo = kc * kRanks;
        const int rank = static_cast<int>(J->rank);
        const int64_t tokens = J->tokens;
        if constexpr (SRC == RCH_SRC_U8) {
            const int64_t rs = J->src_row_stride, cs = J->src_col_stride;
            const bool vec = (J->flags & RCH_JF_SRC_VEC) != 0;
            constexpr int kGroups = kRanks / 16;                       // 16-byte groups per token row
            constexpr int kIters = (kTileTokens * kGroups + kThreads - 1) / kThreads;
            if (vec && k_lo + kRanks <= rank && t0 + kTileTokens <= tokens) {
                // Full tile, aligned rows: every thread issues all its 16-byte loads before any
                // LDS write, so their latencies overlap.
                u4 bytes[kIters];
#pragma unroll
                for (int i = 0; i < kIters; ++i) {
                    const int q = tid + i * kThreads;
                    const int token = q / kGroups, g = q - token * kGroups;
                    if (q < kTileTokens * kGroups) bytes[i] = *gin<u4>(J->src_ptr + (t0 + token) * rs + k_lo + 16 * g);
                }
#pragma unroll
                for (int i = 0; i < kIters; ++i) {
                    const int q = tid + i * kThreads;
                    const int token = q / kGroups, g = q - token * kGroups;
                    if (q < kTileTokens * kGroups) {
                        u2* dst = reinterpret_cast<u2*>(codes + token * kPitch + 16 * g);
                        dst[0] = u2{bytes[i][0], bytes[i][1]};
                        dst[1] = u2{bytes[i][2], bytes[i][3]};
                    }
                }
            } else {
                for (int q = tid; q < kTileTokens * kGroups; q += kThreads) {
                    const int token = q / kGroups, g = q - token * kGroups;
                    const int64_t tt = t0 + token;
                    const int k0 = k_lo + 16 * g;
                    uint32_t w[4] = {0u, 0u, 0u, 0u};
                    if (tt < tokens) {
                        for (int i = 0; i < 16 && k0 + i < rank; ++i)
                            w[i >> 2] |= static_cast<uint32_t>(gin<uint8_t>(J->src_ptr)[tt * rs + (k0 + i) * cs])
                                         << (8 * (i & 3));
                    }
                    u2* dst = reinterpret_cast<u2*>(codes + token * kPitch + 16 * g);
                    dst[0] = u2{w[0], w[1]};
                    dst[1] = u2{w[2], w[3]};
                }
            }
        } else {  // pictures: one thread per (token, half of the rank columns), 16 gathers in flight
            const int token = tid >> 1, half = tid & 1;
            const int64_t tt = t0 + token;
            uint8_t* row = codes + token * kPitch;
            const bool live = tt < tokens;
            const Coords c = coords(J, live ? static_cast<int>(tt) : 0);
            for (int base = half; base < kRanks; base += 32) {
                uint8_t got[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int kl = base + 2 * i;
                    const int k = k_lo + kl;
                    got[i] = (live && kl < kRanks && k < rank) ? gin<uint8_t>(J->src_ptr)[picture_offset(J, k, c)] : 0;
                }
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (base + 2 * i < kRanks) row[base + 2 * i] = got[i];
            }
        }
        for (int i = tid; i < kRanks; i += kThreads) {
            const int k = k_lo + i;
            affine[i] = k < rank ? __fmul_rn(gin<float>(J->scale_ptr)[k], pre) : 0.0f;
            affine[kRanks + i] = k < rank ? __fmul_rn(gin<float>(J->offset_ptr)[k], pre) : 0.0f;
        }
    };

    CoefFrag<PREC> cf[KS];
    auto build = [&](const rch_job* J, int t0, int kc) {
        if constexpr (kStaged) {
            __syncthreads();  // earlier readers of codes / affine are done
            stage(J, t0, kc);
            __syncthreads();
            const uint8_t* row = codes + (wave * 32 + col) * kPitch;
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                float a[8];
                if constexpr (PREC == RCH_PREC_FP32) {
                    const u2 b0 = *reinterpret_cast<const u2*>(row + 16 * s);  // rows are 8-byte aligned
                    const u2 b1 = *reinterpret_cast<const u2*>(row + 16 * s + 8);
                    const u4 b = {b0[0], b0[1], b1[0], b1[1]};
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int kl = 2 * j + h;
                        a[j] = dequant((b[kl >> 2] >> (8 * (kl & 3))) & 0xffu, affine[16 * s + kl],
                                       affine[kRanks + 16 * s + kl]);
                    }
                } else {
                    const int kl = 16 * s + 8 * h;
                    const u2 b = *reinterpret_cast<const u2*>(row + kl);
                    const f4 sc0 = *reinterpret_cast<const f4*>(affine + kl);
                    const f4 sc1 = *reinterpret_cast<const f4*>(affine + kl + 4);
                    const f4 of0 = *reinterpret_cast<const f4*>(affine + kRanks + kl);
                    const f4 of1 = *reinterpret_cast<const f4*>(affine + kRanks + kl + 4);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        a[j] = dequant((b[0] >> (8 * j)) & 0xffu, sc0[j], of0[j]);
                        a[j + 4] = dequant((b[1] >> (8 * j)) & 0xffu, sc1[j], of1[j]);
                    }
                }
                if (!valid) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) a[j] = 0.0f;
                }
                set_frag_scaled(cf[s], a);  // the prescale is in the staged affine
            }
        } else {  // float coefficients, read per lane and used as is
            const int rank = static_cast<int>(J->rank);
            const int dtype = static_cast<int>(J->src_dtype);
            const int64_t row = t * J->src_row_stride;
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                float a[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int k = (kc * KS + s) * 16 + k_slot<PREC>(h, j);
                    a[j] = (valid && k < rank) ? load_value(J->src_ptr, row + k * J->src_col_stride, dtype) : 0.0f;
                }
                set_frag(cf[s], a, pre);
            }
        }
    };

    f16v acc = {};
    fetch(0);
    commit(0, 0);
    __syncthreads();
    for (int st = 0; st < steps; ++st) {
        const int buffer = st & 1;
        int tile, block, kc;
        locate(st, tile, block, kc);
        // The job is re-derived from the restrict descriptor table every step: its fields are
        // then uniform scalar loads instead of per-lane vector loads.
        const rch_job* J = jobs + tiles[2 * tile];
        if (st + 1 < steps) fetch(st + 1);
        if (CHUNKED || tile != current) {
            if (tile != current) {
                t = tiles[2 * tile + 1] + wave * 32 + col;
                valid = t < J->tokens;
                xy = coords(J, valid ? static_cast<int>(t) : 0);
                // Power-of-two prescale of the coefficients (fp16 modes), undone in the epilogue.
                coef_exp = kFp16 ? static_cast<int>(J->coef_exp) : 0;
                if (kFp16 && J->bound_index >= 0) coef_exp = prescale_exponent(__int_as_float(scratch[J->bound_index]));
                pre = pow2f(coef_exp);
                current = tile;
            }
            build(J, tiles[2 * tile + 1], kc);
        }
        const int c0 = block * 32 + 16 * h;
        const int rope = static_cast<int>(J->rope);
        const bool store = (!CHUNKED || kc == nk - 1) && valid && c0 < channels;
        RopeRegs rr;
        rr.vec = false;
        if (store && rope != RCH_ROPE_NONE) rr = load_rope(J, rope, c0, head_dim, t, xy.f, xy.y, xy.x);
        if (kc == 0) acc = f16v{};
#pragma unroll
        for (int s = 0; s < KS; ++s) acc = mfma_step<PREC>(&lds[buffer][s * kStepFrags + lane * kFrag], cf[s], acc);
        // Commit the next step's fragments before this step's stores: on gfx9 stores and loads
        // share vmcnt and complete in order, so waiting for the fetched fragments after issuing
        // the stores would also wait for the stores to reach memory.
        if (st + 1 < steps) commit(st + 1, buffer ^ 1);
        if (store) {
            // Undo the coefficient prescale and the block exponent of the packed basis (per
            // 32-channel block, written by the packer): one exact power-of-two scaling.
            const int e = coef_exp + scratch[J->basis_exp_index + block];
            float v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = __builtin_amdgcn_ldexpf(acc[i], -e);
            if (rope != RCH_ROPE_NONE) {
                if (rr.vec) {
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        rotate(v[2 * p], v[2 * p + 1], rr.c0[p], rr.s0[p]);
                        rotate(v[8 + 2 * p], v[8 + 2 * p + 1], rr.c1[p], rr.s1[p]);
                    }
                } else {
                    apply_rope(J, rope, v, c0, channels, head_dim, t, xy.f, xy.y, xy.x);
                }
            }
            store16(J, v, c0, channels, head_dim, t, out_dtype);
        }
        __syncthreads();
    }
}

}  // namespace

// Kernel arguments: jobs, tiles, bounds, scratch words, pack_base (added to every rch_job.pack_ptr),
// rank chunks, channels, head_dim, output dtype.
typedef void (*RestoreFn)(const rch_job*, const int32_t*, const int32_t*, const int32_t*, int64_t, int, int, int, int);

// A compiled variant: kernel, its register-resident rank steps and whether it chunks the rank.
struct RestoreVariant {
    RestoreFn fn;
    int ks;
    bool chunked;
};

namespace {

// Largest KS (16-rank steps) whose coefficient fragments stay in registers without spills.
template <int PREC> constexpr int kMaxSteps = PREC == RCH_PREC_FP32 ? 8 : (PREC == RCH_PREC_FP16X2 ? 12 : 16);

template <int PREC, int SRC>
RestoreVariant pick_ks(int ks) {
    if constexpr (PREC == RCH_PREC_FP32) {
        if (ks <= 4) return {restore_kernel<PREC, SRC, 4, false>, 4, false};
        if (ks <= 8) return {restore_kernel<PREC, SRC, 8, false>, 8, false};
        return {restore_kernel<PREC, SRC, 8, true>, 8, true};
    } else {
        if (ks <= 2) return {restore_kernel<PREC, SRC, 2, false>, 2, false};
        if (ks <= 4) return {restore_kernel<PREC, SRC, 4, false>, 4, false};
        if (ks <= 8) return {restore_kernel<PREC, SRC, 8, false>, 8, false};
        if (ks <= 12) return {restore_kernel<PREC, SRC, 12, false>, 12, false};
        if (ks <= kMaxSteps<PREC>) return {restore_kernel<PREC, SRC, kMaxSteps<PREC>, false>, kMaxSteps<PREC>, false};
        return {restore_kernel<PREC, SRC, 8, true>, 8, true};
    }
}

template <int PREC>
RestoreVariant pick_source(int source_kind, int ks) {
    switch (source_kind) {
        case RCH_SRC_FLOAT: return pick_ks<PREC, RCH_SRC_FLOAT>(ks);
        case RCH_SRC_U8: return pick_ks<PREC, RCH_SRC_U8>(ks);
        case RCH_SRC_PICTURE: return pick_ks<PREC, RCH_SRC_PICTURE>(ks);
        default: return {nullptr, 0, false};
    }
}

}  // namespace

// One per precision translation unit (restore_<precision>.hip).
RestoreVariant pick_restore_fp32(int source_kind, int ks);
RestoreVariant pick_restore_fp16(int source_kind, int ks);
RestoreVariant pick_restore_fp16x2(int source_kind, int ks);
RestoreVariant pick_restore_bf16(int source_kind, int ks);

}  // namespace rch
