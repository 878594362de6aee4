#pragma once
// Fast variant of the fused restore kernel (restore_kernel.h) for the common serving case:
// fp16 / fp16x2 / bf16 products, uint8 (16-byte aligned rows) or picture codes, head_dim a
// multiple of 32, destinations with unit dim stride and 16-byte aligned rows, slots and RoPE
// tables under 2 GiB.  The host routes a launch group here only when every job qualifies
// (RCH_GF_FAST); everything else runs restore_kernel.
//
// Same fragments, products and epilogue arithmetic as restore_kernel (identical bits); only
// the schedule differs:
//   * Every per-step memory access is a buffer instruction.  Lanes and steps that fall outside
//     a job get an out-of-range offset (loads return zero, stores are dropped) instead of a
//     branch, so a step is straight-line code with a fixed sequence of memory operations and
//     the compiler waits for exactly the loads it needs.
//   * gfx9 loads and stores share one in-order counter: waiting for a load also waits for
//     every older store.  Basis fragments are fetched two steps ahead (register ring -> LDS
//     buffer -> product) and RoPE values one step ahead, so no wait covers the stores of the
//     step just finished.
//   * Inside a tile the 32-channel blocks are walked position-major (dim block 0 of every
//     head, then dim block 1, ...), so consecutive steps of a lane use the same RoPE rows.
//   * Per-lane destination offsets and RoPE row offsets are computed once per tile; the
//     (tile, dim block, head) cursor advances incrementally (no divisions per step).
#include "restore_kernel.h"

namespace rch {
namespace {

struct Cursor {
    int tile, bp, head;
};

// Three resident workgroups per CU where the LDS footprint allows it (KS <= 12: at most
// 51 KB each) and the step fits the 168-VGPR budget that implies without spills (the two
// RoPE pair sets add 32 VGPRs, so RoPE variants get three only up to KS = 8).  Head-pair steps
// (HP = 2) hold two accumulators and twice the staged fragments: two workgroups.
template <int KS, bool ROPE, int HP>
constexpr int kFastOccupancy = HP == 2 ? 2 : (((KS <= 12 && !ROPE) || (KS <= 8 && ROPE)) ? 3 : 2);

// LDS and fragment geometry of one straight-line variant.
template <int PREC, int KS, int HP, int SPLIT>
struct FastGeometry {
    static constexpr int kThreadsT = kThreads * SPLIT;  // threads of the workgroup
    static constexpr int kStepFrags = 64;               // u4 fragments of one 16-rank step of one block
    static constexpr int kHeadFrags = KS * kStepFrags;  // fragments of one block (one head)
    static constexpr int kBuffer = HP * kHeadFrags;     // u4 fragments of one step's LDS buffer
    static constexpr int kRanks = KS * 16;
    static constexpr int kPitch = kRanks + 8;
    // Rank halves: the high half's partial sums of a step, [step parity][token group][16][64 lanes]
    // fp32, share the codes buffer (codes are read only between the barriers of a tile entry).
    static constexpr int kReduceBytes = SPLIT == 2 ? 2 * 4 * 16 * 64 * 4 : 0;
    static constexpr int kCodesBytes = kTileTokens * kPitch > kReduceBytes ? kTileTokens * kPitch : kReduceBytes;
};

// LDS of a straight-line launch: two step buffers of basis fragments, the staged codes (or the
// rank halves' partial sums), the staged affine and the picture cell offsets.
struct FastLds {
    u4* lds;
    uint8_t* codes;
    float* affine;
    int64_t* cell_offset;
};

// HP = heads per step: 1, or 2 (RCH_GF_HEAD_PAIRS, an even head count): a step then computes the
// same 32-channel dim block of two adjacent heads, so the per-step bookkeeping, barrier and
// waits are shared by twice the matrix work and each RoPE pair set serves both heads.
// SPLIT = rank halves: 1, or 2 (RCH_GF_SPLIT_RANK, ranks beyond one wave's registers): the
// workgroup has 8 waves, waves w and w + 4 hold the coefficient fragments of the same 32 tokens
// for the low and the high half of the rank steps, each computes its half of every block's
// product, and the high half hands its fp32 partial sums to the low half through LDS, which
// adds them and runs the epilogue (the only difference from one chain: the fp32 summation
// order of the two halves).
//
// One workgroup's part of a launch: work units [first_unit, first_unit + steps) of the tile
// table (unit u: tile u / (blocks per tile), then dim block and head).
template <int PREC, int KS, bool ROPE, int OUT, int HP, int SPLIT>
__device__ __forceinline__ void fast_range(const rch_job* __restrict__ jobs, const int32_t* __restrict__ tiles,
                                           const int first_unit, const int steps,
                                           const int32_t* __restrict__ scratch, int64_t pack_base, int heads,
                                           int head_dim, const FastLds& shared) {
    static_assert(PREC != RCH_PREC_FP32, "the fp32 mode runs restore_kernel");
    static_assert(HP == 1 || HP == 2, "one or two heads per step");
    static_assert(SPLIT == 1 || (SPLIT == 2 && HP == 1 && KS % 8 == 0), "rank halves: one head per step");
    using G = FastGeometry<PREC, KS, HP, SPLIT>;
    constexpr int kThreadsT = G::kThreadsT;
    constexpr int kKsWave = KS / SPLIT;                  // rank steps held by one wave
    constexpr int kStepFrags = G::kStepFrags;
    constexpr int kHeadFrags = G::kHeadFrags;
    constexpr int kBuffer = G::kBuffer;
    constexpr int kPer = kBuffer / kThreadsT;
    static_assert(kBuffer % kThreadsT == 0, "KS must be a multiple of 4: every thread moves whole fragments");
    constexpr int kRanks = G::kRanks;
    constexpr int kPitch = G::kPitch;
    constexpr bool kFp16 = PREC == RCH_PREC_FP16 || PREC == RCH_PREC_FP16X2;
    constexpr int kEsize = OUT == RCH_DT_F32 ? 4 : 2;
    u4* const lds = shared.lds;
    uint8_t* const codes = shared.codes;
    float* const affine = shared.affine;
    int64_t* const cell_offset = shared.cell_offset;

    if (steps <= 0) return;
    const int head_blocks = head_dim >> 5;
    const int head_steps = heads / HP;  // steps per dim block
    const int per_tile = head_steps * head_blocks;  // work units per tile (blocks / HP)
    const int last_tile = (first_unit + steps - 1) / per_tile;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, h = lane >> 5, col = lane & 31;
    const int group = wave & 3;      // token group: tokens 32 group .. 32 group + 31 of the tile
    const int half = wave >> 2;      // rank half (SPLIT == 2), else 0

    // Unit u of a tile is (dim block u / head_steps, first head HP * (u % head_steps)).  Prefetch
    // cursors past the range end stay on the range's last tile (their fragments are fetched and
    // never used).
    auto advance = [&](Cursor c) __attribute__((always_inline)) {
        c.head += HP;
        const bool next_bp = c.head == heads;
        c.head = next_bp ? 0 : c.head;
        c.bp += next_bp ? 1 : 0;
        const bool next_tile = c.bp == head_blocks;
        c.bp = next_tile ? 0 : c.bp;
        c.tile = min(c.tile + (next_tile ? 1 : 0), last_tile);
        return c;
    };

    // Basis fragments of a step: thread loads fragments q = tid + i * 256 of the step's block(s)
    // (head j = q / kHeadFrags of the step; zero beyond the job's rank).  The pack of the fetched
    // tile's job and this thread's offsets within a block column are set up only when the fetch
    // cursor enters a new tile; a step adds the first block's offset (out-of-range offsets stay
    // out of range: the block offset is below 2^31).
    int fetch_tile = -1;
    uint32_t fetch_lane[kPer];
    __amdgpu_buffer_rsrc_t pack = make_rsrc(0, 0);
    auto fetch = [&](const Cursor& c, u4 (&into)[kPer]) __attribute__((always_inline)) {
        if (c.tile != fetch_tile) {
            const rch_job* J = jobs + tiles[2 * c.tile];
            const int ks = static_cast<int>((J->rank + 15) >> 4);
            const int nblocks = static_cast<int>(J->pack_nblocks);
            pack = make_rsrc(pack_base + J->pack_ptr, int64_t(ks) * nblocks * 1024);
#pragma unroll
            for (int i = 0; i < kPer; ++i) {
                const int q = tid + i * kThreadsT;
                const int j = q / kHeadFrags, s = (q % kHeadFrags) >> 6, li = q & 63;
                fetch_lane[i] = s < ks ? static_cast<uint32_t>(s * nblocks + j * head_blocks) * 1024u + li * 16
                                       : kOutOfRange;
            }
            fetch_tile = c.tile;
        }
        const uint32_t block_offset = static_cast<uint32_t>((c.head * head_blocks + c.bp) * 1024);
#pragma unroll
        for (int i = 0; i < kPer; ++i)
            into[i] = __builtin_amdgcn_raw_buffer_load_b128(pack, fetch_lane[i] + block_offset, 0, 0);
    };
    auto commit = [&](int buffer, const u4 (&from)[kPer]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) lds[buffer * kBuffer + tid + i * kThreadsT] = from[i];
    };

    // Per-lane state of the current tile.
    uint32_t dst_lane = kOutOfRange;  // byte offset of this lane's 16 channels of (token, head 0, dim 0)
    uint32_t row_t = 0, row_h = 0, row_w = 0;  // byte offsets of this token's RoPE rows
    __amdgpu_buffer_rsrc_t dst = make_rsrc(0, 0), pairs = make_rsrc(0, 0);
    int coef_exp = 0, sec0 = 0, sec1 = 0, head_bytes = 0;
    int bexp_base = 0;  // first scratch word of the tile's basis block exponents
    CoefFrag<PREC> cf[kKsWave];

    f4 rope_next[4], rope_now[4];  // RoPE pairs of the next / current dim block

    // (cos, sin) of this lane's 8 pairs j = j0 .. j0 + 7 of a dim block (j0 = 16 bp + 8 h):
    // into[p] = (cos, sin) of pairs j0 + 2p and j0 + 2p + 1.  A pair's table row depends on its
    // section.  Dim blocks whose pairs all keep their section across each load's two pairs use
    // four 16-byte loads; a block where a section boundary splits such a load (Wan: the odd
    // boundary, one block per head) loads its pairs one by one.  The test is uniform.
    auto rope_load = [&](int bp, f4 (&into)[4]) __attribute__((always_inline)) {
        const int jb = 16 * bp;
        // Row of pair j: row_t, plus (row_h - row_t) from section 1 on, plus (row_w - row_h) from
        // section 2 on (written as adds of selected deltas: a three-way select of the rows is
        // turned into a lookup table in scratch memory).
        const uint32_t rt = row_t, d1 = row_h - row_t, d2 = row_w - row_h;
        const int s0 = __builtin_amdgcn_readfirstlane(sec0), s1 = __builtin_amdgcn_readfirstlane(sec1);
        auto row_of = [&](int j) __attribute__((always_inline)) {
            return rt + (j >= s0 ? d1 : 0u) + (j >= s1 ? d2 : 0u);
        };
        // An odd section boundary inside [jb, jb + 16) splits a two-pair load.
        const bool split = ((s0 & 1) && s0 > jb && s0 < jb + 16) || ((s1 & 1) && s1 > jb && s1 < jb + 16);
        const int j0 = jb + 8 * h;
        if (!split) {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const int j = j0 + 2 * p;
                into[p] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(pairs, row_of(j) + static_cast<uint32_t>(j * 8), 0, 0));
            }
        } else {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const int j = j0 + 2 * p;
                const u2 a = __builtin_amdgcn_raw_buffer_load_b64(pairs, row_of(j) + static_cast<uint32_t>(j * 8), 0, 0);
                const u2 b = __builtin_amdgcn_raw_buffer_load_b64(pairs, row_of(j + 1) + static_cast<uint32_t>((j + 1) * 8), 0, 0);
                into[p] = f4{__uint_as_float(a[0]), __uint_as_float(a[1]), __uint_as_float(b[0]), __uint_as_float(b[1])};
            }
        }
    };

    // Tile entry: stage the tile's codes and affine in LDS, convert this wave's 32 tokens to
    // coefficient fragments.  All waves passed a barrier since they last read codes / affine
    // (rank halves: the low half reads partial sums after the step barrier, so the entry starts
    // with a barrier of its own).
    auto enter = [&](const rch_job* J, int t0, int first_bp) __attribute__((always_inline)) {
        if constexpr (SPLIT == 2) __syncthreads();
        const int64_t tokens = J->tokens;
        const int64_t t = t0 + group * 32 + col;
        const bool valid = t < tokens;
        const Coords xy = coords(J, valid ? static_cast<int>(t) : 0);
        dst = make_rsrc(J->dst_ptr, J->dst_bytes);
        dst_lane = valid ? static_cast<uint32_t>((t * J->dst_token_stride + 16 * h) * kEsize) : kOutOfRange;
        if constexpr (ROPE) {
            const int64_t row_bytes = J->rope_row_stride * 8;  // interleaved (cos, sin) fp32 pairs
            pairs = make_rsrc(J->pairs_ptr, J->pairs_bytes);
            // Dense tables: every pair uses row row_t + t.
            const bool dense = J->rope == RCH_ROPE_DENSE;
            const uint32_t first = static_cast<uint32_t>((J->row_t + (dense ? t : int64_t(xy.f))) * row_bytes);
            const uint32_t second = static_cast<uint32_t>((J->row_h + xy.y) * row_bytes);
            const uint32_t third = static_cast<uint32_t>((J->row_w + xy.x) * row_bytes);
            row_t = first;
            row_h = dense ? first : second;
            row_w = dense ? first : third;
            sec0 = static_cast<int>(J->sec_t);
            sec1 = static_cast<int>(J->sec_t + J->sec_h);
            // Pairs of the tile's first dim block, issued before the code loads so that the
            // drain below covers them.
            rope_load(first_bp, rope_now);
        }
        coef_exp = kFp16 ? static_cast<int>(J->coef_exp) : 0;
        head_bytes = static_cast<int>(J->dst_head_stride) * kEsize;
        const float pre = pow2f(coef_exp);  // folded into the staged affine
        const int rank = static_cast<int>(J->rank);
        bexp_base = static_cast<int>(J->basis_exp_index);
        if (SPLIT == 2 || J->pic_slots == 0) {  // uint8 rows, 16-byte aligned (rank halves: uint8 rows only)
            const int64_t rs = J->src_row_stride;
            constexpr int kGroups = kRanks / 16;
            constexpr int kIters = (kTileTokens * kGroups + kThreadsT - 1) / kThreadsT;
            const __amdgpu_buffer_rsrc_t src = make_rsrc(J->src_ptr + t0 * rs, (tokens - t0) * rs);
            // Rank halves: the thread index made opaque here, so the staging offsets are
            // recomputed per tile instead of being hoisted out of the tile loop (and spilled).
            int me = tid;
            if constexpr (SPLIT == 2) asm volatile("" : "+v"(me));
            u4 bytes[kIters];
#pragma unroll
            for (int i = 0; i < kIters; ++i) {
                const int q = me + i * kThreadsT;
                const int token = q / kGroups, g = q - token * kGroups;
                const uint32_t offset = (q < kTileTokens * kGroups && 16 * g < rank)
                                            ? static_cast<uint32_t>(token * rs + 16 * g)
                                            : kOutOfRange;
                bytes[i] = __builtin_amdgcn_raw_buffer_load_b128(src, offset, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < kIters; ++i) {
                const int q = me + i * kThreadsT;
                const int token = q / kGroups, g = q - token * kGroups;
                if (q < kTileTokens * kGroups) {
                    // Bytes past the rank (row padding) are staged as they are: their affine
                    // entries are zero, so they dequantize to 0 * q + 0 = 0.
                    const u4 b = bytes[i];
                    u2* out = reinterpret_cast<u2*>(codes + token * kPitch + 16 * g);
                    out[0] = u2{b[0], b[1]};
                    out[1] = u2{b[2], b[3]};
                }
            }
        } else if (J->pic_slots >= rank) {
            // Pictures of one segment (channel_tiles.v1: rank column k in cell k of every frame's
            // picture).  The cells' offsets within a picture are tabulated in LDS; then thread
            // (token, p) gathers the columns of blocks [32 b + 16 p, + 16) of its token: a wave's
            // lanes are 64 consecutive tokens, so each byte load of one column reads contiguous
            // runs of a cell row, and a block's 16 loads are in flight together.
            for (int k = tid; k < kRanks; k += kThreadsT) {
                const int planes = static_cast<int>(J->pic_planes), cols = static_cast<int>(J->pic_grid_cols);
                const int plane = k % planes, index = k / planes;
                const int cell_row = index / cols, cell_col = index - cell_row * cols;
                cell_offset[k] = plane * J->pic_plane_stride + static_cast<int64_t>(cell_row) * J->grid_h * J->pic_row_stride +
                                 static_cast<int64_t>(cell_col) * J->grid_w;
            }
            __syncthreads();
            const RCH_GLOBAL uint8_t* base = gin<uint8_t>(J->src_ptr);
            if (J->flags & RCH_JF_PIC_VEC4) {
                // Aligned geometry: thread (quad, part) loads tokens 4 quad .. + 3 (one cell-row word:
                // x % 4 == 0 and grid_w % 4 == 0 keep them in one row) of ranks 4 g .. 4 g + 3 for the
                // groups g of its part, and transposes the 4 x 4 bytes into 4 tokens' rank words.
                constexpr int kQuads = kTileTokens / 4, kParts4 = kThreadsT / kQuads;
                const int quad = tid % kQuads, part = tid / kQuads;
                const int64_t tt = t0 + 4 * quad;
                const bool live = tt < tokens;  // tokens % 4 == 0: a quad is whole or past the end
                const Coords c = coords(J, live ? static_cast<int>(tt) : 0);
                const int64_t lane = gin<int64_t>(J->pic_table_ptr)[c.f] + c.y * J->pic_row_stride + c.x;
#pragma unroll
                for (int g = part; 4 * g < kRanks; g += kParts4) {
                    uint32_t d[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int k = 4 * g + r;
                        const bool take = live & (k < rank);
                        d[r] = *reinterpret_cast<const RCH_GLOBAL uint32_t*>(base + (take ? lane + cell_offset[k] : 0));
                        d[r] = take ? d[r] : 0u;  // word 0 of the first picture is readable
                    }
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const uint32_t word = ((d[0] >> (8 * t)) & 0xffu) | (((d[1] >> (8 * t)) & 0xffu) << 8) |
                                              (((d[2] >> (8 * t)) & 0xffu) << 16) | (((d[3] >> (8 * t)) & 0xffu) << 24);
                        *reinterpret_cast<uint32_t*>(codes + (4 * quad + t) * kPitch + 4 * g) = word;
                    }
                }
            } else {
                const int token = tid & (kTileTokens - 1), p = tid / kTileTokens;  // p is wave-uniform
                constexpr int kParts = kThreadsT / kTileTokens;
                const int64_t tt = t0 + token;
                const bool live = tt < tokens;
                const Coords c = coords(J, live ? static_cast<int>(tt) : 0);
                const int64_t lane = gin<int64_t>(J->pic_table_ptr)[c.f] + c.y * J->pic_row_stride + c.x;
                uint8_t* row = codes + token * kPitch;
                for (int b = p; 16 * b < kRanks; b += kParts) {
                    uint32_t got[16];
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int k = 16 * b + i;
                        const bool take = live & (k < rank);
                        got[i] = base[take ? lane + cell_offset[k] : 0];  // byte 0 of the first picture is readable
                        got[i] = take ? got[i] : 0u;
                    }
                    u4 word;
#pragma unroll
                    for (int w = 0; w < 4; ++w)
                        word[w] = got[4 * w] | (got[4 * w + 1] << 8) | (got[4 * w + 2] << 16) | (got[4 * w + 3] << 24);
                    u2* out = reinterpret_cast<u2*>(row + 16 * b);
                    out[0] = u2{word[0], word[1]};
                    out[1] = u2{word[2], word[3]};
                }
            }
        } else {  // pictures of several segments: one thread per (token, half of the rank columns)
            const int token = tid >> 1, half = tid & 1;
            const int64_t tt = t0 + token;
            uint8_t* row = codes + token * kPitch;
            const bool live = tt < tokens;
            const Coords c = coords(J, live ? static_cast<int>(tt) : 0);
            for (int base = half; base < kRanks; base += 32) {
                uint8_t got[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int k = base + 2 * i;
                    got[i] = (live && k < kRanks && k < rank) ? gin<uint8_t>(J->src_ptr)[picture_offset(J, k, c)] : 0;
                }
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (base + 2 * i < kRanks) row[base + 2 * i] = got[i];
            }
        }
        for (int i = tid; i < kRanks; i += kThreadsT) {
            affine[i] = i < rank ? __fmul_rn(gin<float>(J->scale_ptr)[i], pre) : 0.0f;
            affine[kRanks + i] = i < rank ? __fmul_rn(gin<float>(J->offset_ptr)[i], pre) : 0.0f;
        }
        __syncthreads();
        const uint8_t* mine = codes + (group * 32 + col) * kPitch;
#pragma unroll
        for (int s = 0; s < kKsWave; ++s) {
            int kl = 16 * (half * kKsWave + s) + 8 * h;
            // Rank halves hold 12-16 fragments per wave: a step's LDS reads wait for the previous
            // step's fragment (ordered asm statements), or the hoisted reads of later steps spill.
            if constexpr (SPLIT == 2) asm volatile("" : "+v"(kl));
            const u2 b = *reinterpret_cast<const u2*>(mine + kl);
            const f4 sc0 = *reinterpret_cast<const f4*>(affine + kl);
            const f4 sc1 = *reinterpret_cast<const f4*>(affine + kl + 4);
            const f4 of0 = *reinterpret_cast<const f4*>(affine + kRanks + kl);
            const f4 of1 = *reinterpret_cast<const f4*>(affine + kRanks + kl + 4);
            // Lanes past the job's tokens convert whatever codes they staged: only their own
            // (never stored) output columns depend on them.
            float a[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                a[j] = dequant((b[0] >> (8 * j)) & 0xffu, sc0[j], of0[j]);
                a[j + 4] = dequant((b[1] >> (8 * j)) & 0xffu, sc1[j], of1[j]);
            }
            set_frag_scaled(cf[s], a);
            if constexpr (SPLIT == 2) asm volatile("" ::"v"(cf[s].hi));
        }
        if constexpr (SPLIT == 2) __syncthreads();  // codes are read; the steps reuse them for partial sums
    };

    // Epilogue of head x of a step: undo the exponents, RoPE, cast, store this lane's 16 channels.
    auto epilogue = [&](const Cursor& c, int x, const f16v& acc, const f4 (&rope)[4], int block_e) __attribute__((always_inline)) {
        // Undo the coefficient prescale and the block's basis exponent (exact powers of two).
        const int e = coef_exp + block_e;
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = __builtin_amdgcn_ldexpf(acc[i], -e);
        if constexpr (ROPE) {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                rotate(v[4 * p], v[4 * p + 1], rope[p][0], rope[p][1]);
                rotate(v[4 * p + 2], v[4 * p + 3], rope[p][2], rope[p][3]);
            }
        }
        const uint32_t at = dst_lane + static_cast<uint32_t>((c.head + x) * head_bytes + c.bp * 32 * kEsize);
        if constexpr (OUT == RCH_DT_F32) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f4 out = {v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, out), dst, at + 16 * q, 0, 0);
            }
        } else if constexpr (OUT == RCH_DT_BF16) {
            bf8 a, b;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                a[i] = static_cast<__bf16>(v[i]);
                b[i] = static_cast<__bf16>(v[i + 8]);
            }
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, a), dst, at, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, b), dst, at + 16, 0, 0);
        } else {
            h8 a, b;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                a[i] = static_cast<_Float16>(v[i]);
                b[i] = static_cast<_Float16>(v[i + 8]);
            }
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, a), dst, at, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, b), dst, at + 16, 0, 0);
        }
    };

    // One step: products of the staged block(s) over this wave's rank steps, then the epilogue;
    // ends with the step barrier (after which the LDS buffer of this step may be refilled).
    auto finish = [&](const Cursor& c, int buffer, const f4 (&rope)[4]) __attribute__((always_inline)) {
        // Basis fragments are read from LDS three steps ahead of their products (a rotating
        // window of four registers per head).
        constexpr int kAhead = kKsWave < 3 ? kKsWave : 3;
        const u4* frags = lds + buffer * kBuffer + lane + half * kKsWave * kStepFrags;
        u4 window[HP][kAhead + 1];
#pragma unroll
        for (int j = 0; j < kAhead; ++j) {
#pragma unroll
            for (int x = 0; x < HP; ++x) window[x][j] = frags[x * kHeadFrags + j * kStepFrags];
        }
        // Basis block exponents of the step's blocks: scalar loads (they do not queue behind the
        // vector stores of earlier steps), issued before the products and used by the epilogue.
        int block_e[HP];
#pragma unroll
        for (int x = 0; x < HP; ++x) block_e[x] = scratch[bexp_base + (c.head + x) * head_blocks + c.bp];
        if constexpr (HP == 2) {
            // Head 0's products, then head 1's products with head 0's epilogue placed between
            // them: its VALU work and stores issue while the matrix pipe works on head 1.
            f16v a0 = f16v{}, a1 = f16v{};
            u4 next[kAhead + 1];
#pragma unroll
            for (int j = 0; j < kAhead; ++j) next[j] = frags[kHeadFrags + j * kStepFrags];
#pragma unroll
            for (int s = 0; s < kKsWave; ++s) {
                if (s + kAhead < kKsWave) window[0][(s + kAhead) % (kAhead + 1)] = frags[(s + kAhead) * kStepFrags];
                a0 = mfma_frag<PREC>(window[0][s % (kAhead + 1)], cf[s], a0);
            }
            __builtin_amdgcn_sched_barrier(0);  // keep the two product chains apart
#pragma unroll
            for (int s = 0; s < kKsWave; ++s) {
                if (s + kAhead < kKsWave) next[(s + kAhead) % (kAhead + 1)] = frags[kHeadFrags + (s + kAhead) * kStepFrags];
                a1 = mfma_frag<PREC>(next[s % (kAhead + 1)], cf[s], a1);
            }
            epilogue(c, 0, a0, rope, block_e[0]);
            // Up to six VALU instructions of head 0's epilogue after each product of head 1.
            constexpr int kProducts = PREC == RCH_PREC_FP16X2 ? 2 * kKsWave : kKsWave;
#pragma unroll
            for (int i = 0; i < kProducts; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // VALU
            }
            epilogue(c, 1, a1, rope, block_e[1]);
            __syncthreads();
            return;
        }
        f16v acc[HP];
#pragma unroll
        for (int x = 0; x < HP; ++x) acc[x] = f16v{};
#pragma unroll
        for (int s = 0; s < kKsWave; ++s) {
#pragma unroll
            for (int x = 0; x < HP; ++x) {
                if (s + kAhead < kKsWave) window[x][(s + kAhead) % (kAhead + 1)] = frags[x * kHeadFrags + (s + kAhead) * kStepFrags];
                acc[x] = mfma_frag<PREC>(window[x][s % (kAhead + 1)], cf[s], acc[x]);
            }
        }
        if constexpr (SPLIT == 1) {
#pragma unroll
            for (int x = 0; x < HP; ++x) epilogue(c, x, acc[x], rope, block_e[x]);
            __syncthreads();
        } else {
            // Partial sums of the high half, lane-contiguous per accumulator element (one
            // 4-byte LDS word per lane and element: no bank conflicts).
            float* partial = reinterpret_cast<float*>(codes) + ((buffer * 4 + group) * 16) * 64 + lane;
            if (half == 1) {
#pragma unroll
                for (int i = 0; i < 16; ++i) partial[i * 64] = acc[0][i];
            }
            __syncthreads();
            if (half == 0) {
                f16v sum = acc[0];
#pragma unroll
                for (int i = 0; i < 16; ++i) sum[i] += partial[i * 64];
                epilogue(c, 0, sum, rope, block_e[0]);
            }
        }
    };

    // Cursors of steps st (now), st + 1 and st + 2.
    Cursor now;
    {
        now.tile = first_unit / per_tile;
        const int local = first_unit - now.tile * per_tile;
        now.bp = local / head_steps;
        now.head = (local - now.bp * head_steps) * HP;
    }
    Cursor ahead1 = advance(now), ahead2 = advance(ahead1);
    u4 ring[kPer];

    fetch(now, ring);
    commit(0, ring);
    fetch(ahead1, ring);
    // Loops: tile (entry: stage and convert the tile's coefficients; its loads drain the memory
    // counter) > dim block (RoPE pairs change) > head (the steps: straight-line code whose only
    // predecessors are the loop entry and its own back edge, so the waits the compiler places
    // are the steady-state ones).  In step st the ring holds the fragments of step st + 1
    // (fetched during step st - 1); they go to the other LDS buffer and the fragments of step
    // st + 2 are fetched in their place.
    int st = 0;
    while (st < steps) {
        const int tile = now.tile;
        enter(jobs + tiles[2 * tile], tiles[2 * tile + 1], now.bp);
        while (st < steps && now.tile == tile) {
            // RoPE pairs of the next dim block are fetched at the start of this one and copied at
            // the end of its last step: the wait before the copy follows a fixed number of memory
            // operations (it covers loads only; waiting for a store to complete costs
            // microseconds under this write stream), and the loads have the whole dim block to
            // arrive (a load queues behind the stores issued before it).
            if constexpr (ROPE) {
                if (now.bp + 1 < head_blocks) rope_load(now.bp + 1, rope_next);
            }
            const int run = min((heads - now.head) / HP, steps - st);
            for (int i = 0; i < run; ++i, ++st) {
                commit((st + 1) & 1, ring);
                fetch(ahead2, ring);
                finish(now, st & 1, rope_now);  // ends with the step barrier
                if constexpr (ROPE) {
                    if (i + 1 == run) {
#pragma unroll
                        for (int p = 0; p < 4; ++p) rope_now[p] = rope_next[p];
                    }
                }
                now = ahead1;
                ahead1 = ahead2;
                ahead2 = advance(ahead2);
            }
        }
    }
}

// One launch group: workgroup b runs units [bounds[b'], bounds[b' + 1]) (b' = XCD-swizzled index).
template <int PREC, int KS, bool ROPE, int OUT, int HP, int SPLIT>
__global__ void __launch_bounds__(kThreads * SPLIT, (SPLIT == 2 ? 1 : kFastOccupancy<KS, ROPE, HP>))
restore_fast_kernel(const rch_job* __restrict__ jobs, const int32_t* __restrict__ tiles,
                    const int32_t* __restrict__ bounds, const int32_t* __restrict__ scratch, int64_t pack_base,
                    int heads, int head_dim) {
    using G = FastGeometry<PREC, KS, HP, SPLIT>;
    __shared__ u4 lds[2 * G::kBuffer];
    __shared__ __attribute__((aligned(16))) uint8_t codes[G::kCodesBytes];
    __shared__ __attribute__((aligned(16))) float affine[2 * G::kRanks];
    __shared__ int64_t cell_offset[G::kRanks];  // pictures: byte offset of rank column k's cell in a picture
    const int range = xcd_unit(blockIdx.x, gridDim.x);
    const int first_unit = bounds[range];
    fast_range<PREC, KS, ROPE, OUT, HP, SPLIT>(jobs, tiles, first_unit, bounds[range + 1] - first_unit, scratch,
                                               pack_base, heads, head_dim, FastLds{lds, codes, affine, cell_offset});
}

// Two head-pair launch groups of one call in one persistent launch: the tile table holds the
// first group's tiles (RoPE, KS0 rank steps) and then the second's (no RoPE, KS1 steps); units
// below split_unit (the first group's tiles x blocks per tile) run the first variant, the others
// the second, and one cost-balanced split of the concatenated units covers both.  One grid ramps
// up and drains once per call instead of once per group; each unit's arithmetic is the single
// group kernel's, so the output bits are the same.
template <int PREC, int OUT, int KS0, int KS1>
__global__ void __launch_bounds__(kThreads, 2)
restore_pair_kernel(const rch_job* __restrict__ jobs, const int32_t* __restrict__ tiles,
                    const int32_t* __restrict__ bounds, const int32_t* __restrict__ scratch, int64_t pack_base,
                    int heads, int head_dim, int split_unit) {
    using G0 = FastGeometry<PREC, KS0, 2, 1>;
    using G1 = FastGeometry<PREC, KS1, 2, 1>;
    constexpr int kBuffer = G0::kBuffer > G1::kBuffer ? G0::kBuffer : G1::kBuffer;
    constexpr int kCodes = G0::kCodesBytes > G1::kCodesBytes ? G0::kCodesBytes : G1::kCodesBytes;
    constexpr int kRanks = G0::kRanks > G1::kRanks ? G0::kRanks : G1::kRanks;
    __shared__ u4 lds[2 * kBuffer];
    __shared__ __attribute__((aligned(16))) uint8_t codes[kCodes];
    __shared__ __attribute__((aligned(16))) float affine[2 * kRanks];
    __shared__ int64_t cell_offset[kRanks];
    const FastLds shared{lds, codes, affine, cell_offset};
    const int range = xcd_unit(blockIdx.x, gridDim.x);
    const int begin = bounds[range], end = bounds[range + 1];
    // Every step of a range ends with a workgroup barrier, so the second variant may refill the
    // LDS the first one used as soon as it starts.
    const int end0 = min(end, split_unit), begin1 = max(begin, split_unit);
    fast_range<PREC, KS0, true, OUT, 2, 1>(jobs, tiles, begin, end0 - begin, scratch, pack_base, heads, head_dim,
                                            shared);
    fast_range<PREC, KS1, false, OUT, 2, 1>(jobs, tiles, begin1, end - begin1, scratch, pack_base, heads, head_dim,
                                             shared);
}

// Kernel arguments: jobs, tiles, bounds, scratch words, pack_base (added to every rch_job.pack_ptr:
// 0 for absolute fragment addresses), heads, head_dim.
typedef void (*FastFn)(const rch_job*, const int32_t*, const int32_t*, const int32_t*, int64_t, int, int);
typedef void (*PairFn)(const rch_job*, const int32_t*, const int32_t*, const int32_t*, int64_t, int, int, int);

// Work-unit shape of a straight-line launch.
enum FastShape : int { kOneHead = 0, kHeadPairs = 1, kRankHalves = 2 };

template <int PREC, bool ROPE, int OUT, int HP>
FastFn fast_ks(int ks, int* chosen) {
    if (ks <= 4) { *chosen = 4; return restore_fast_kernel<PREC, 4, ROPE, OUT, HP, 1>; }
    if (ks <= 8) { *chosen = 8; return restore_fast_kernel<PREC, 8, ROPE, OUT, HP, 1>; }
    if (ks <= 12) { *chosen = 12; return restore_fast_kernel<PREC, 12, ROPE, OUT, HP, 1>; }
    if constexpr (PREC != RCH_PREC_FP16X2 && HP == 1) {
        if (ks <= 16) { *chosen = 16; return restore_fast_kernel<PREC, 16, ROPE, OUT, HP, 1>; }
    }
    *chosen = 0;
    return nullptr;
}

// Rank halves: the rank steps beyond the one-wave variants, up to 32 (512 ranks).
template <int PREC, bool ROPE, int OUT>
FastFn split_ks(int ks, int* chosen) {
    if constexpr (PREC == RCH_PREC_FP16X2) {
        if (ks <= 16) { *chosen = 16; return restore_fast_kernel<PREC, 16, ROPE, OUT, 1, 2>; }
    }
    if (ks <= 24) { *chosen = 24; return restore_fast_kernel<PREC, 24, ROPE, OUT, 1, 2>; }
    if (ks <= 32) { *chosen = 32; return restore_fast_kernel<PREC, 32, ROPE, OUT, 1, 2>; }
    *chosen = 0;
    return nullptr;
}

template <int PREC, bool ROPE, int OUT>
FastFn fast_shape(int ks, int shape, int* chosen) {
    switch (shape) {
        case kOneHead: return fast_ks<PREC, ROPE, OUT, 1>(ks, chosen);
        case kHeadPairs: return fast_ks<PREC, ROPE, OUT, 2>(ks, chosen);
        case kRankHalves: return split_ks<PREC, ROPE, OUT>(ks, chosen);
        default: *chosen = 0; return nullptr;
    }
}

template <int PREC, int OUT>
FastFn fast_rope(int ks, bool rope, int shape, int* chosen) {
    return rope ? fast_shape<PREC, true, OUT>(ks, shape, chosen) : fast_shape<PREC, false, OUT>(ks, shape, chosen);
}

template <int PREC>
FastFn pick_fast(int ks, bool rope, int out_dtype, int shape, int* chosen) {
    switch (out_dtype) {
        case RCH_DT_F32: return fast_rope<PREC, RCH_DT_F32>(ks, rope, shape, chosen);
        case RCH_DT_F16: return fast_rope<PREC, RCH_DT_F16>(ks, rope, shape, chosen);
        case RCH_DT_BF16: return fast_rope<PREC, RCH_DT_BF16>(ks, rope, shape, chosen);
        default: *chosen = 0; return nullptr;
    }
}

template <int PREC, int OUT, int KS0>
PairFn pair_second(int ks1, int* chosen1) {
    if (ks1 <= 4) { *chosen1 = 4; return restore_pair_kernel<PREC, OUT, KS0, 4>; }
    if (ks1 <= 8) { *chosen1 = 8; return restore_pair_kernel<PREC, OUT, KS0, 8>; }
    if (ks1 <= 12) { *chosen1 = 12; return restore_pair_kernel<PREC, OUT, KS0, 12>; }
    *chosen1 = 0;
    return nullptr;
}

template <int PREC, int OUT>
PairFn pair_first(int ks0, int ks1, int* chosen0, int* chosen1) {
    if (ks0 <= 4) { *chosen0 = 4; return pair_second<PREC, OUT, 4>(ks1, chosen1); }
    if (ks0 <= 8) { *chosen0 = 8; return pair_second<PREC, OUT, 8>(ks1, chosen1); }
    if (ks0 <= 12) { *chosen0 = 12; return pair_second<PREC, OUT, 12>(ks1, chosen1); }
    *chosen0 = *chosen1 = 0;
    return nullptr;
}

// The pair kernel of a (RoPE group, plain group) of head-pair units, or nullptr (bf16 and f16
// outputs, up to 12 rank steps per group).
template <int PREC>
PairFn pick_pair(int ks0, int ks1, int out_dtype, int* chosen0, int* chosen1) {
    *chosen0 = *chosen1 = 0;
    switch (out_dtype) {
        case RCH_DT_F16: return pair_first<PREC, RCH_DT_F16>(ks0, ks1, chosen0, chosen1);
        case RCH_DT_BF16: return pair_first<PREC, RCH_DT_BF16>(ks0, ks1, chosen0, chosen1);
        default: return nullptr;
    }
}

}  // namespace

// One per precision translation unit (restore_<precision>.hip); nullptr when no fast variant
// of that work-unit shape (FastShape) covers the rank.
FastFn pick_fast_fp16(int ks, bool rope, int out_dtype, int shape, int* chosen);
FastFn pick_fast_fp16x2(int ks, bool rope, int out_dtype, int shape, int* chosen);
FastFn pick_fast_bf16(int ks, bool rope, int out_dtype, int shape, int* chosen);

// Pair kernels (restore_pair_fp16x2.hip): fp16x2 products.
PairFn pick_pair_fp16x2(int ks0, int ks1, int out_dtype, int* chosen0, int* chosen1);

}  // namespace rch
