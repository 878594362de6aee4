#pragma once
// Channel-slice variant of the fused restore kernel (restore_kernel.h) for uint8 codes in
// 16-byte aligned rows, the fp16 / fp16x2 / bf16 products and head_dim % 32 == 0 (the common
// serving case; the host routes other launch groups to restore_fast.h or restore_kernel.h).
//
// Same fragments, products and epilogue arithmetic as restore_kernel (identical bits); the work
// is organised around the MI355X's costs instead:
//   * A workgroup (4 waves; two workgroups per CU, so each SIMD runs one wave of each and their
//     independent phases hide each other's latencies) owns a slice of at most 8 32-channel
//     blocks (whole heads) and walks a contiguous range of 32-token tiles with its 4 waves in
//     lockstep.  Each wave owns two blocks of the slice (two heads, one dim block) and keeps
//     their basis fragments in registers for the whole range.
//   * A tile's codes are dequantized once per workgroup, 8 ranks of one token per item and the
//     same number of items per thread, into fp16 (hi, lo) fragments in an LDS tile that every
//     wave reads, so one fragment read feeds the products of both of a wave's blocks.  The LDS
//     tiles are double buffered, and each iteration computes tile T, finishes tile T - 1 and
//     dequantizes tile T + 1 (independent work the scheduler interleaves with the products);
//     one barrier per tile (an LDS wait, no store drain) separates the buffers.
//   * Every global load of the steady state is issued ahead of its use in straight-line code:
//     a tile's codes two tiles ahead, its RoPE pairs one tile ahead, into registers that
//     alternate between the two halves of a two-tile loop body.  The wait before each use then
//     counts only older operations, never the stores of the tile just written (loads and stores
//     share one in-order counter on gfx9).
// Work is balanced per workgroup by the host: entry e of workgroup w (wg_entries[w] <= e <
// wg_entries[w + 1]) covers tiles [tile0 + u0, tile0 + u1) of one (basis, head slice) pair.
#include "restore_fast.h"

namespace rch {
namespace {

constexpr int kSliceWaves = 4;                 // two workgroups share a CU (one wave of each per SIMD)
constexpr int kSliceThreads = 64 * kSliceWaves;
constexpr int kSliceBlocks = 2 * kSliceWaves;  // 32-channel blocks per slice: two per wave
constexpr int kSliceJobs = 8;                  // jobs whose affine one entry stages in LDS

static_assert(sizeof(rch_slice_entry) == 32, "rch_slice_entry is 8 x int32");

template <int PREC, int KS, bool ROPE, int OUT>
__global__ void __launch_bounds__(kSliceThreads, 2)
restore_slice_kernel(const rch_job* __restrict__ jobs, const int32_t* __restrict__ tiles,
                     const rch_slice_entry* __restrict__ entries, const int32_t* __restrict__ wg_entries,
                     const int32_t* __restrict__ scratch, int head_dim) {
    static_assert(PREC != RCH_PREC_FP32, "the fp32 mode runs restore_kernel");
    constexpr int kItems = 2 * KS * 32 / kSliceThreads;  // 8-rank dequantization items per thread and tile
    static_assert(kItems * kSliceThreads == 2 * KS * 32, "every thread dequantizes the same number of items");
    constexpr bool kSplit = PREC == RCH_PREC_FP16X2;
    constexpr bool kFp16 = PREC == RCH_PREC_FP16 || kSplit;
    constexpr int kParts = kSplit ? 2 : 1;  // fragment planes: hi (and lo)
    constexpr int kRanks = 16 * KS;
    constexpr int kEsize = OUT == RCH_DT_F32 ? 4 : 2;
    constexpr int kMfmas = 2 * kParts * KS;          // products per wave and tile
    constexpr int kValuPerMfma = ROPE ? 11 : 6;      // VALU slots interleaved after each
    // Coefficient fragments of two tiles, [step][plane][lane]; two arrays (not one indexed by
    // parity) so the compiler knows a tile's reads never alias the next tile's writes.
    __shared__ u4 coef0[KS][kParts][64];
    __shared__ u4 coef1[KS][kParts][64];
    __shared__ __attribute__((aligned(16))) float affine[kSliceJobs][2][kRanks];

    const int tid = threadIdx.x;
    // The wave index is uniform; saying so keeps per-wave values in scalar registers.
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, h = lane >> 5, col = lane & 31;
    const int wg = xcd_unit(blockIdx.x, gridDim.x);
    const int head_blocks = head_dim >> 5;
    // Dequantization items: item q = tid + i * threads is ranks 8 (q / 32) .. + 7 of token q % 32,
    // one fragment lane of one step (consecutive threads write consecutive LDS fragments).
    const int dq_token = tid & 31, dq_half0 = tid >> 5;

    for (int e = wg_entries[wg]; e < wg_entries[wg + 1]; ++e) {
        const rch_slice_entry E = entries[e];
        const int nh = E.nh, nh_pad = E.nh + (E.nh & 1);
        // Never planned by the host; uniform, so no barrier is skipped unevenly.
        if (nh <= 0 || nh_pad * head_blocks > kSliceBlocks || E.u0 >= E.u1) continue;
        __syncthreads();  // the previous entry's LDS readers are done
        const int t_begin = E.tile0 + E.u0, t_end = E.tile0 + E.u1;

        // This wave's blocks: dim block bp of slice heads hw and hw + 1.
        const int pairs = nh_pad >> 1;
        const int bp = wave / pairs, hw = 2 * (wave - bp * pairs);
        const bool have0 = bp < head_blocks && hw < nh, have1 = bp < head_blocks && hw + 1 < nh;
        const rch_job* P = jobs + E.pack_job;
        const int64_t nblocks = P->pack_nblocks;
        const __amdgpu_buffer_rsrc_t pack = make_rsrc(P->pack_ptr, int64_t(E.pack_ksteps) * nblocks * 1024);
        const int blk0 = (E.head0 + hw) * head_blocks + bp, blk1 = blk0 + head_blocks;
        u4 basis0[KS], basis1[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const bool step = s < E.pack_ksteps;
            basis0[s] = __builtin_amdgcn_raw_buffer_load_b128(
                pack, (have0 && step) ? static_cast<uint32_t>((s * nblocks + blk0) * 1024 + lane * 16) : kOutOfRange, 0, 0);
            basis1[s] = __builtin_amdgcn_raw_buffer_load_b128(
                pack, (have1 && step) ? static_cast<uint32_t>((s * nblocks + blk1) * 1024 + lane * 16) : kOutOfRange, 0, 0);
        }
        const int bexp0 = have0 ? scratch[P->basis_exp_index + blk0] : 0;
        const int bexp1 = have1 ? scratch[P->basis_exp_index + blk1] : 0;

        // The affine (scale | offset) of the entry's jobs in LDS, one slot per job in tile order,
        // zero beyond each job's rank (those codes contribute 0).
        {
            int slot = 0, last = -1;
            for (int t = t_begin; t < t_end; ++t) {
                const int j = tiles[2 * t];
                if (j == last) continue;
                last = j;
                if (slot < kSliceJobs) {
                    const rch_job* J = jobs + j;
                    const int rank = static_cast<int>(J->rank);
                    const RCH_GLOBAL float* scale = gin<float>(J->scale_ptr);
                    const RCH_GLOBAL float* offset = gin<float>(J->offset_ptr);
                    // The power-of-two coefficient prescale (fp16 modes) is folded in here.
                    const float pre = pow2f(kFp16 ? static_cast<int>(J->coef_exp) : 0);
                    for (int i = tid; i < kRanks; i += kSliceThreads) {
                        affine[slot][0][i] = i < rank ? __fmul_rn(scale[i], pre) : 0.0f;
                        affine[slot][1][i] = i < rank ? __fmul_rn(offset[i], pre) : 0.0f;
                    }
                }
                ++slot;
            }
        }
        __syncthreads();  // the prologue dequantizes with affine entries staged by other waves

        // Tiles past the range clamp to its last tile (their loads are out of range).
        auto tile_job = [&](int t) __attribute__((always_inline)) { return tiles[2 * min(t, t_end - 1)]; };

        // This thread's codes of tile t, 8 per item (zero past the range, the job's tokens or its
        // rank; non-short-circuit conditions and selects keep the loop body branch-free).
        auto load_codes = [&](int t, u2 (&into)[kItems]) __attribute__((always_inline)) {
            const int tc = min(t, t_end - 1);
            const rch_job* J = jobs + tiles[2 * tc];
            const int64_t t0 = tiles[2 * tc + 1];
            const int64_t rs = J->src_row_stride, rank = J->rank;
            const __amdgpu_buffer_rsrc_t src = make_rsrc(J->src_ptr + t0 * rs, (J->tokens - t0) * rs);
#pragma unroll
            for (int i = 0; i < kItems; ++i) {
                const int half = dq_half0 + i * (kSliceThreads / 32);
                const bool live = (t < t_end) & (8 * half < rank);
                const uint32_t offset = static_cast<uint32_t>(dq_token * rs + 8 * half);
                into[i] = __builtin_amdgcn_raw_buffer_load_b64(src, live ? offset : kOutOfRange, 0, 0);
            }
        };

        // Dequantize this thread's items of tile t (affine slot `slot`) into the LDS tile `coef`:
        // fragment lane (token, h) of step s holds ranks 16 s + 8 h .. + 7.
        auto dequant = [&](int t, int slot, const u2 (&codes)[kItems], u4 (&coef)[KS][kParts][64])
                           __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < kItems; ++i) {
                const int half = dq_half0 + i * (kSliceThreads / 32);
                const float* sc = &affine[slot][0][8 * half];
                const float* of = &affine[slot][1][8 * half];
                const f4 s0 = *reinterpret_cast<const f4*>(sc);
                const f4 s1 = *reinterpret_cast<const f4*>(sc + 4);
                const f4 o0 = *reinterpret_cast<const f4*>(of);
                const f4 o1 = *reinterpret_cast<const f4*>(of + 4);
                float a[8];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    a[j] = rch::dequant((codes[i][0] >> (8 * j)) & 0xffu, s0[j], o0[j]);
                    a[j + 4] = rch::dequant((codes[i][1] >> (8 * j)) & 0xffu, s1[j], o1[j]);
                }
                CoefFrag<PREC> f;
                set_frag_scaled(f, a);
                u4* out = &coef[half >> 1][0][32 * (half & 1) + dq_token];
                out[0] = __builtin_bit_cast(u4, f.hi);
                if constexpr (kSplit) out[64] = __builtin_bit_cast(u4, f.lo);
            }
        };

        // Per-lane RoPE table rows of this lane's token in tile t (byte offsets).
        struct Rows {
            uint32_t t, h, w;
        };
        auto rope_rows = [&](int t) __attribute__((always_inline)) {
            Rows r = {0u, 0u, 0u};
            if constexpr (ROPE) {
                const int tc = min(t, t_end - 1);
                const rch_job* J = jobs + tiles[2 * tc];
                const int64_t tok = tiles[2 * tc + 1] + col, tokens = J->tokens;
                const Coords xy = coords(J, tok < tokens ? static_cast<int>(tok) : 0);
                const int64_t row_bytes = J->rope_row_stride * 8;  // interleaved (cos, sin) fp32 pairs
                const bool dense = J->rope == RCH_ROPE_DENSE;
                const int64_t row_t = J->row_t, row_h = J->row_h, row_w = J->row_w;  // loaded unconditionally
                r.t = static_cast<uint32_t>((row_t + (dense ? tok : int64_t(xy.f))) * row_bytes);
                const uint32_t rh = static_cast<uint32_t>((row_h + xy.y) * row_bytes);
                const uint32_t rw = static_cast<uint32_t>((row_w + xy.x) * row_bytes);
                r.h = dense ? r.t : rh;
                r.w = dense ? r.t : rw;
            }
            return r;
        };

        // (cos, sin) of this lane's pairs j0 .. j0 + 7 of dim block bp (j0 = 16 bp + 8 h) for the
        // token rows `r` of tile t: one 8-byte load per pair from the row of the pair's section,
        // branch-free (a fixed number of loads keeps the steady-state wait counts exact).
        auto rope_load = [&](int t, const Rows& r, f4 (&into)[4]) __attribute__((always_inline)) {
            if constexpr (ROPE) {
                const rch_job* J = jobs + tile_job(t);
                const __amdgpu_buffer_rsrc_t pairs = make_rsrc(J->pairs_ptr, t < t_end ? J->pairs_bytes : 0);
                const int s0 = static_cast<int>(J->sec_t), s1 = static_cast<int>(J->sec_t + J->sec_h);
                const uint32_t d1 = r.h - r.t, d2 = r.w - r.h;
                const int j0 = 16 * bp + 8 * h;
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const int j = j0 + 2 * p;
                    const uint32_t ra = r.t + (j >= s0 ? d1 : 0u) + (j >= s1 ? d2 : 0u);
                    const uint32_t rb = r.t + (j + 1 >= s0 ? d1 : 0u) + (j + 1 >= s1 ? d2 : 0u);
                    const u2 a = __builtin_amdgcn_raw_buffer_load_b64(pairs, ra + static_cast<uint32_t>(j * 8), 0, 0);
                    const u2 b = __builtin_amdgcn_raw_buffer_load_b64(pairs, rb + static_cast<uint32_t>((j + 1) * 8), 0, 0);
                    into[p] = f4{__uint_as_float(a[0]), __uint_as_float(a[1]), __uint_as_float(b[0]), __uint_as_float(b[1])};
                }
            }
        };

        // Undo the prescales (exact powers of two), RoPE, cast, store one block of tile t.
        auto epilogue = [&](const f16v& acc, int ex, const f4 (&rope)[4], const __amdgpu_buffer_rsrc_t& dst,
                            uint32_t offset) __attribute__((always_inline)) {
            float v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = __builtin_amdgcn_ldexpf(acc[i], -ex);
            if constexpr (ROPE) {
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    rotate(v[4 * p], v[4 * p + 1], rope[p][0], rope[p][1]);
                    rotate(v[4 * p + 2], v[4 * p + 3], rope[p][2], rope[p][3]);
                }
            }
            if constexpr (OUT == RCH_DT_F32) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const f4 out = {v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, out), dst, offset + 16 * q, 0, 0);
                }
            } else if constexpr (OUT == RCH_DT_BF16) {
                bf8 lo, hi;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    lo[i] = static_cast<__bf16>(v[i]);
                    hi[i] = static_cast<__bf16>(v[i + 8]);
                }
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, lo), dst, offset, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, hi), dst, offset + 16, 0, 0);
            } else {
                h8 lo, hi;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    lo[i] = static_cast<_Float16>(v[i]);
                    hi[i] = static_cast<_Float16>(v[i + 8]);
                }
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, lo), dst, offset, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, hi), dst, offset + 16, 0, 0);
            }
        };

        // Products of one tile (LDS tile `coef`) for both of this wave's blocks.
        auto products = [&](const u4 (&coef)[KS][kParts][64], f16v& acc0, f16v& acc1) __attribute__((always_inline)) {
            acc0 = f16v{};
            acc1 = f16v{};
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                CoefFrag<PREC> c;
                if constexpr (PREC == RCH_PREC_BF16) {
                    c.hi = __builtin_bit_cast(bf8, coef[s][0][lane]);
                } else {
                    c.hi = __builtin_bit_cast(h8, coef[s][0][lane]);
                    if constexpr (kSplit) c.lo = __builtin_bit_cast(h8, coef[s][kParts - 1][lane]);
                }
                acc0 = mfma_frag<PREC>(basis0[s], c, acc0);
                acc1 = mfma_frag<PREC>(basis1[s], c, acc1);
            }
        };

        // Epilogues of tile t's two blocks (nothing is stored for t before the range).
        auto finish = [&](int t, const f16v& acc0, const f16v& acc1, const f4 (&rope)[4]) __attribute__((always_inline)) {
            const int tc = max(t, t_begin);
            const rch_job* J = jobs + tiles[2 * tc];
            const int64_t tok = tiles[2 * tc + 1] + col;
            const __amdgpu_buffer_rsrc_t dst = make_rsrc(J->dst_ptr, J->dst_bytes);
            const int64_t tokens = J->tokens, token_stride = J->dst_token_stride;
            const uint32_t offset = static_cast<uint32_t>((tok * token_stride + 16 * h) * kEsize);
            const uint32_t lane_offset = ((t >= t_begin) & (tok < tokens)) ? offset : kOutOfRange;
            const int head_bytes = static_cast<int>(J->dst_head_stride) * kEsize;
            const uint32_t base = lane_offset + static_cast<uint32_t>((E.head0 + hw) * head_bytes + bp * 32 * kEsize);
            const int coef_exp = kFp16 ? static_cast<int>(J->coef_exp) : 0;
            epilogue(acc0, coef_exp + bexp0, rope, dst, have0 ? base : kOutOfRange);
            epilogue(acc1, coef_exp + bexp1, rope, dst, have1 ? base + static_cast<uint32_t>(head_bytes) : kOutOfRange);
        };

        // Prologue: tile t_begin dequantized into coef0 and tile t_begin + 1's codes in registers
        // (nothing stored yet, so the wait is short).
        int dq_job = tile_job(t_begin), dq_slot = 0;
        u2 codes_a[kItems], codes_b[kItems];
        f4 rope_a[4], rope_b[4];
        f16v acc_a0 = {}, acc_a1 = {}, acc_b0 = {}, acc_b1 = {};
#pragma unroll
        for (int p = 0; p < 4; ++p) rope_b[p] = f4{};
        load_codes(t_begin, codes_a);
        load_codes(t_begin + 1, codes_b);
        wait_vector_memory();
        dequant(t_begin, 0, codes_a, coef0);
        __syncthreads();

        // Iteration t (three tiles in flight, every step independent of the others, so the
        // scheduler can fill the matrix-core shadows with the VALU work): prefetch tile t + 2's
        // codes and tile t's RoPE pairs, dequantize tile t + 1 into the other LDS tile, compute
        // tile t, finish tile t - 1 (its accumulators and pairs from the previous iteration),
        // barrier.  The `_a` / `_b` registers and the two LDS tiles alternate between the two
        // halves of the loop body.
        auto iteration = [&](int t, const u4 (&coef_read)[KS][kParts][64], u4 (&coef_write)[KS][kParts][64],
                             const u2 (&codes_use)[kItems], u2 (&codes_next)[kItems], f4 (&rope_now)[4],
                             const f4 (&rope_prev)[4],
                             f16v& acc0, f16v& acc1, const f16v& prev0, const f16v& prev1) __attribute__((always_inline)) {
            load_codes(t + 2, codes_next);
            rope_load(t, rope_rows(t), rope_now);
            const int j1 = tile_job(t + 1);
            dq_slot = j1 != dq_job ? min(dq_slot + 1, kSliceJobs - 1) : dq_slot;
            dq_job = j1;
            dequant(t + 1, dq_slot, codes_use, coef_write);
            products(coef_read, acc0, acc1);
            finish(t - 1, prev0, prev1, rope_prev);
            // Spread the VALU work (dequantization, epilogues) between the products: each MFMA
            // is followed by a few independent VALU instructions that issue under it.
#pragma unroll
            for (int i = 0; i < kMfmas; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, kValuPerMfma, 0);  // VALU
            }
            __syncthreads();
        };
        int t = t_begin;
        for (; t + 1 < t_end; t += 2) {
            iteration(t, coef0, coef1, codes_b, codes_a, rope_a, rope_b, acc_a0, acc_a1, acc_b0, acc_b1);
            iteration(t + 1, coef1, coef0, codes_a, codes_b, rope_b, rope_a, acc_b0, acc_b1, acc_a0, acc_a1);
        }
        if (t < t_end) {
            iteration(t, coef0, coef1, codes_b, codes_a, rope_a, rope_b, acc_a0, acc_a1, acc_b0, acc_b1);
            finish(t, acc_a0, acc_a1, rope_a);
        } else {
            finish(t - 1, acc_b0, acc_b1, rope_b);
        }
    }
}

typedef void (*SliceFn)(const rch_job*, const int32_t*, const rch_slice_entry*, const int32_t*, const int32_t*, int);

template <int PREC, bool ROPE, int OUT>
SliceFn slice_ks(int ks, int* chosen, int* max_blocks) {
    if (ks <= 4) { *chosen = 4; *max_blocks = kSliceBlocks; return restore_slice_kernel<PREC, 4, ROPE, OUT>; }
    if (ks <= 8) { *chosen = 8; *max_blocks = kSliceBlocks; return restore_slice_kernel<PREC, 8, ROPE, OUT>; }
    if (ks <= 12) { *chosen = 12; *max_blocks = kSliceBlocks; return restore_slice_kernel<PREC, 12, ROPE, OUT>; }
    if constexpr (PREC != RCH_PREC_FP16X2) {
        if (ks <= 16) { *chosen = 16; *max_blocks = kSliceBlocks; return restore_slice_kernel<PREC, 16, ROPE, OUT>; }
    }
    *chosen = 0;
    *max_blocks = 0;
    return nullptr;
}

template <int PREC>
SliceFn pick_slice(int ks, bool rope, int out_dtype, int* chosen, int* max_blocks) {
    switch (out_dtype) {
        case RCH_DT_F32: return rope ? slice_ks<PREC, true, RCH_DT_F32>(ks, chosen, max_blocks) : slice_ks<PREC, false, RCH_DT_F32>(ks, chosen, max_blocks);
        case RCH_DT_F16: return rope ? slice_ks<PREC, true, RCH_DT_F16>(ks, chosen, max_blocks) : slice_ks<PREC, false, RCH_DT_F16>(ks, chosen, max_blocks);
        case RCH_DT_BF16: return rope ? slice_ks<PREC, true, RCH_DT_BF16>(ks, chosen, max_blocks) : slice_ks<PREC, false, RCH_DT_BF16>(ks, chosen, max_blocks);
        default: *chosen = 0; *max_blocks = 0; return nullptr;
    }
}

}  // namespace

// One per precision translation unit (restore_<precision>.hip); nullptr when no slice variant
// covers the rank.  max_blocks = the 32-channel blocks one slice workgroup holds.
SliceFn pick_slice_fp16(int ks, bool rope, int out_dtype, int* chosen, int* max_blocks);
SliceFn pick_slice_fp16x2(int ks, bool rope, int out_dtype, int* chosen, int* max_blocks);
SliceFn pick_slice_bf16(int ks, bool rope, int out_dtype, int* chosen, int* max_blocks);

}  // namespace rch
