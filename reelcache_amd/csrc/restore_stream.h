#pragma once
// Basis-stationary restore kernel for uint8 code rows (MI355X, gfx950).
//
// Arithmetic (the fp16x2 mode, folded): with codes q, per-rank scale s and offset o, the
// restored value is  sum_k (q_k s_k + o_k) Q_kc = sum_k (q_k - 128) W_kc + b_c  with
// W_kc = s_k Q_kc and b_c = sum_k (o_k + 128 s_k) Q_kc.  The codes enter the MFMA as exact fp16
// integers (q - 128), W is split into an fp16 head and tail (2^e W = hi + lo, 22 significant
// bits, e a power-of-two prescale per 32-channel block), and b is an FP64 sum rounded once.
// Both products accumulate in fp32, exactly like the reference's two fp16 products per rank
// step (reelcache/restore_kernels.py:1497-1513); the product's rounding differs from the
// reference's dequantize-then-split order only far inside its error bound (:1208-1227).
//
// Work decomposition:
//   * A work unit is (job, head, 32-token tile); head_dim is 128, so a workgroup's four waves
//     each own one 32-channel block of the head.  Units run job-major, then head, then tile, and
//     a persistent workgroup walks a contiguous unit range, so a wave's block of W (both
//     fp16 parts, 8 VGPRs per 16 ranks), its bias and exponent stay in registers for many units.
//   * W, b and e come from a per-(job, block) slab written by scaled_pack_kernel (restore.hip).
//   * The tile's codes are loaded one unit ahead (coalesced 16-byte rows), converted to fp16
//     B-operand fragments (two v_perm + two packed fp16 subtractions per 4 codes) and written
//     to double-buffered LDS; each wave reads its fragments with one 16-byte LDS read per
//     rank step.  RoPE (cos, sin) pairs of the tile are gathered into LDS the same way.
//   * out^T[c, t] = W^T[c, k] (q - 128)[k, t] on v_mfma_f32_32x32x16_f16: channels on the MFMA
//     rows (permuted by block_channel), so each lane's accumulator holds 16 consecutive channels
//     of one token; the epilogue is one fma (2^-e scale + bias: a single rounding), RoPE on
//     interleaved pairs without FMA, one cast and two 16-byte stores per lane.
//   * One workgroup barrier per unit.  Loads for unit u + 1 are issued before unit u's stores,
//     so waiting for them never waits for those stores (gfx9 counts loads and stores in one
//     in-order counter).
#include "restore_kernel.h"

namespace rch {
namespace {

constexpr int kStreamTokens = 32;      // tokens per work unit
constexpr int kFragPitch = 1040;       // bytes between the LDS code fragments of two rank steps (1 KB + 16)
constexpr int kRopePitch = 528;        // bytes between the LDS RoPE rows of two tokens (64 pairs x 8 + 16)
constexpr int kSectionPairs = 2048;    // (cos, sin) pairs of a job's separable table held in LDS

// RoPE modes of the stream kernel: none; separable tables (the job's section rows staged in LDS
// once per job); dense tables (each unit's rows gathered into LDS, one unit ahead).
enum StreamRope : int { kRopeNone = 0, kRopeSections = 1, kRopeDense = 2 };

// Bytes of one (job, 32-channel block) slab written by the pack kernel: KS hi fragments, KS lo
// fragments (64 lanes x 16 bytes each), the block's 32 fp32 biases in channel order and its
// exponent, padded to 256 bytes.
__host__ __device__ constexpr int64_t stream_slab_bytes(int64_t ks) { return (ks * 2048 + 128 + 16 + 255) / 256 * 256; }

// Resident workgroups per CU: the software-pipelined variants (every RoPE mode but dense) hold a
// second accumulator; three workgroups fit only the smallest rank steps.
template <int KS, int ROPE>
constexpr int kStreamOccupancy = ROPE == 2 ? (KS <= 8 ? 3 : 2) : (KS <= 4 ? 3 : 2);

// (frame, row, column) of a token, advanced by whole tiles without divisions.
struct GridPos {
    int f, y, x;
    __device__ __forceinline__ void advance(int by, int width, int height) {
        x += by;
        while (x >= width) {
            x -= width;
            ++y;
        }
        while (y >= height) {
            y -= height;
            ++f;
        }
    }
};

__device__ __forceinline__ GridPos grid_pos(int t, int width, int height) {
    const int plane = width * height;
    GridPos p;
    p.f = t / plane;
    const int rest = t - p.f * plane;
    p.y = rest / width;
    p.x = rest - p.y * width;
    return p;
}

template <int KS, int ROPE, int OUT>
__global__ void __launch_bounds__(kThreads, (kStreamOccupancy<KS, ROPE>))
restore_stream_kernel(const rch_job* __restrict__ jobs, const int32_t* __restrict__ members,
                      const int32_t* __restrict__ bounds, int n_members, int heads, int64_t pack_base) {
    constexpr int kEsize = OUT == RCH_DT_F32 ? 4 : 2;
    constexpr int kChunks = 32 * KS;                               // 16-code chunks of a unit
    constexpr int kIters = (kChunks + kThreads - 1) / kThreads;    // chunks per thread
    __shared__ __attribute__((aligned(16))) uint8_t frags[2][KS * kFragPitch];
    __shared__ __attribute__((aligned(16))) uint8_t rope_lds[ROPE == kRopeDense ? 2 * kStreamTokens * kRopePitch
                                                           : (ROPE == kRopeSections ? 8 * kSectionPairs : 16)];

    const int range = xcd_unit(blockIdx.x, gridDim.x);
    const int first = bounds[range], last = bounds[range + 1];
    if (first >= last) return;
    const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, col = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int stage_token = tid & 31;  // staging: token of this thread's code chunks / RoPE pairs
    const int stage_group = tid >> 5;  // staging: chunk (mod 8) / RoPE pair group of this thread

    // ---- the stager: cursor of the unit being staged and its job's cached fields ----
    int s_member = 0, s_job = 0, s_head = 0, s_t0 = 0;
    int s_tokens = 0, s_rs = 0;
    int64_t s_src = 0, s_bytes = 0;
    uint32_t s_off[kIters];
    int64_t s_rope_row = 0, s_row_bytes = 0, s_pairs = 0, s_pairs_bytes = 0;
    auto stager_job = [&]() __attribute__((always_inline)) {
        const rch_job* J = jobs + s_job;
        s_tokens = static_cast<int>(J->tokens);
        s_rs = static_cast<int>(J->src_row_stride);
        s_src = J->src_ptr;
        s_bytes = J->tokens * J->src_row_stride;
        const int rank = static_cast<int>(J->rank);
#pragma unroll
        for (int i = 0; i < kIters; ++i) {
            const int chunk = stage_group + 8 * i;
            s_off[i] = (chunk < KS && 16 * chunk < rank) ? static_cast<uint32_t>(stage_token * s_rs + 16 * chunk)
                                                         : kOutOfRange;
        }
        if constexpr (ROPE == kRopeDense) {
            s_row_bytes = J->rope_row_stride * 8;
            s_rope_row = J->row_t;
            s_pairs = J->pairs_ptr;
            s_pairs_bytes = J->pairs_bytes;
        }
    };
    {
        int m = 0;
        while (m + 1 < n_members && members[2 * (m + 1)] <= first) ++m;
        const int local = first - members[2 * m];
        const int tiles = (members[2 * (m + 1)] - members[2 * m]) / heads;
        s_member = m;
        s_job = members[2 * m + 1];
        s_head = local / tiles;
        s_t0 = (local - s_head * tiles) * kStreamTokens;
        stager_job();
    }
    auto stager_advance = [&]() __attribute__((always_inline)) {
        s_t0 += kStreamTokens;
        if (s_t0 >= s_tokens) {
            s_t0 = 0;
            if (++s_head == heads) {
                s_head = 0;
                ++s_member;
                if (s_member < n_members) {
                    s_job = members[2 * s_member + 1];
                    stager_job();
                }
            }
        }
    };
    // Codes (and dense RoPE rows) of the stager's unit into registers.
    u4 staged[kIters];
    u4 staged_rope[ROPE == kRopeDense ? 4 : 1];
    auto stage_load = [&]() __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t src = make_rsrc(s_src, s_bytes);
        const uint32_t row = static_cast<uint32_t>(s_t0 * s_rs);
#pragma unroll
        for (int i = 0; i < kIters; ++i)
            staged[i] = __builtin_amdgcn_raw_buffer_load_b128(src, s_off[i] == kOutOfRange ? kOutOfRange : s_off[i] + row,
                                                              0, 0);
        if constexpr (ROPE == kRopeDense) {
            // Pairs 8 g .. 8 g + 7 of the token: one table row per token, 64 contiguous bytes.
            const __amdgpu_buffer_rsrc_t pairs = make_rsrc(s_pairs, s_pairs_bytes);
            const int t = s_t0 + stage_token;
            const uint32_t at = t < s_tokens
                                    ? static_cast<uint32_t>((s_rope_row + t) * s_row_bytes + 64 * stage_group)
                                    : kOutOfRange;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                staged_rope[i] = __builtin_amdgcn_raw_buffer_load_b128(pairs, at == kOutOfRange ? at : at + 16 * i, 0, 0);
        }
    };
    // Codes -> fp16 (q - 128) B fragments: fragment (step s, lane h * 32 + t) holds ranks
    // 16 s + 8 h .. + 7 of token t.  (1024 + q) is built bitwise (0x64 above each code byte) and
    // 1152 subtracted in packed fp16: exact.
    auto stage_store = [&](int buffer) __attribute__((always_inline)) {
        uint8_t* base = frags[buffer];
#pragma unroll
        for (int i = 0; i < kIters; ++i) {
            const int chunk = stage_group + 8 * i;
            if (chunk < KS) {
                const u4 w = staged[i];
                u4 out[2];
#pragma unroll
                for (int half = 0; half < 2; ++half) {
#pragma unroll
                    for (int p = 0; p < 2; ++p) {
                        const uint32_t word = w[2 * half + p];
                        const h2 a = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, word, 0x04010400u)) -
                                     h2{1152.0f16, 1152.0f16};
                        const h2 b = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, word, 0x04030402u)) -
                                     h2{1152.0f16, 1152.0f16};
                        out[half][2 * p] = __builtin_bit_cast(uint32_t, a);
                        out[half][2 * p + 1] = __builtin_bit_cast(uint32_t, b);
                    }
                }
                *reinterpret_cast<u4*>(base + chunk * kFragPitch + stage_token * 16) = out[0];
                *reinterpret_cast<u4*>(base + chunk * kFragPitch + (32 + stage_token) * 16) = out[1];
            }
        }
        if constexpr (ROPE == kRopeDense) {
            uint8_t* row = rope_lds + buffer * kStreamTokens * kRopePitch + stage_token * kRopePitch + 64 * stage_group;
#pragma unroll
            for (int i = 0; i < 4; ++i) *reinterpret_cast<u4*>(row + 16 * i) = staged_rope[i];
        }
    };

    // ---- the consumer: cursor of the unit being computed and its (job, head) state ----
    int c_member = s_member, c_job = s_job, c_head = s_head, c_t0 = s_t0;
    int c_tokens = 0;
    int64_t c_dst = 0, c_dst_bytes = 0;
    uint32_t c_ts = 0;        // bytes between tokens of the destination
    uint32_t c_lane = 0;      // this lane's byte offset of (token c_t0 + col)'s 16 channels
    h8 w_hi[KS], w_lo[KS];
    float bias[16];
    float unscale = 1.0f;
    GridPos pos{0, 0, 0};     // sections RoPE: this lane's token
    int grid_w = 1, grid_h = 1, last_frame = 0, sec0 = 0, sec1 = 0, e_base_h = 0, e_base_w = 0, sec_len_t = 0,
        sec_len_h = 0, sec_len_w = 0;
    // Loads the job's section rows into LDS (all waves; the caller's barrier publishes them).
    auto load_sections = [&](const rch_job* J) __attribute__((always_inline)) {
        const int frames = static_cast<int>(J->frames);
        last_frame = frames - 1;
        grid_h = static_cast<int>(J->grid_h);
        grid_w = static_cast<int>(J->grid_w);
        sec_len_t = static_cast<int>(J->sec_t);
        sec_len_h = static_cast<int>(J->sec_h);
        sec_len_w = 64 - sec_len_t - sec_len_h;
        sec0 = sec_len_t;
        sec1 = sec_len_t + sec_len_h;
        e_base_h = frames * sec_len_t;
        e_base_w = e_base_h + grid_h * sec_len_h;
        const int total = e_base_w + grid_w * sec_len_w;
        const __amdgpu_buffer_rsrc_t pairs = make_rsrc(J->pairs_ptr, J->pairs_bytes);
        const int64_t row_bytes = J->rope_row_stride * 8;
        const int64_t row_t = J->row_t, row_h = J->row_h, row_w = J->row_w;
        for (int p = tid; p < total; p += kThreads) {
            int64_t row;
            int pair;
            if (p < e_base_h) {
                const int r = p / sec_len_t;
                row = row_t + r;
                pair = p - r * sec_len_t;
            } else if (p < e_base_w) {
                const int q = p - e_base_h, r = q / sec_len_h;
                row = row_h + r;
                pair = sec0 + q - r * sec_len_h;
            } else {
                const int q = p - e_base_w, r = q / sec_len_w;
                row = row_w + r;
                pair = sec1 + q - r * sec_len_w;
            }
            const u2 v = __builtin_amdgcn_raw_buffer_load_b64(pairs, static_cast<uint32_t>(row * row_bytes + 8 * pair), 0, 0);
            *reinterpret_cast<u2*>(rope_lds + 8 * p) = v;
        }
    };
    auto consumer_head = [&](bool new_job) __attribute__((always_inline)) {
        const rch_job* J = jobs + c_job;
        if (new_job) {
            c_tokens = static_cast<int>(J->tokens);
            c_dst = J->dst_ptr;
            c_dst_bytes = J->dst_bytes;
            c_ts = static_cast<uint32_t>(J->dst_token_stride * kEsize);
            if constexpr (ROPE == kRopeSections) load_sections(J);
        }
        c_lane = static_cast<uint32_t>((c_head * J->dst_head_stride + 32 * wave + 16 * h) * kEsize) + col * c_ts;
        // This wave's block of W, its biases and exponent, from the job's slab.
        const int64_t slab = pack_base + J->pack_ptr + (c_head * 4 + wave) * stream_slab_bytes(KS);
        const RCH_GLOBAL u4* frag = gin<u4>(slab) + lane;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            w_hi[s] = __builtin_bit_cast(h8, frag[s * 64]);
            w_lo[s] = __builtin_bit_cast(h8, frag[(KS + s) * 64]);
        }
        const RCH_GLOBAL f4* b = gin<f4>(slab + KS * 2048 + 64 * h);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const f4 v = b[q];
            bias[4 * q] = v[0];
            bias[4 * q + 1] = v[1];
            bias[4 * q + 2] = v[2];
            bias[4 * q + 3] = v[3];
        }
        const int e = gin<int32_t>(slab + KS * 2048 + 128)[0];
        // Wait here, on the rare switch: left to the compiler, the wait for these registers
        // lands in the epilogue of every unit, where it also waits for the staged loads.
        wait_vector_memory();
        unscale = pow2f(-e);
        if constexpr (ROPE == kRopeSections) pos = grid_pos(c_t0 + col, grid_w, grid_h);
    };

    // Epilogue of one unit's accumulator: 2^-e scale and bias in one rounding, RoPE, cast, store
    // (nothing is stored for a placeholder, `live` false).
    auto epilogue = [&](const f16v& a, int t0, const GridPos& p, int rope_buffer, bool live) __attribute__((always_inline)) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = __builtin_fmaf(a[i], unscale, bias[i]);
        if constexpr (ROPE == kRopeDense) {
            const uint8_t* row = rope_lds + rope_buffer * kStreamTokens * kRopePitch + col * kRopePitch +
                                 8 * (16 * wave + 8 * h);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f4 cs = *reinterpret_cast<const f4*>(row + 16 * q);  // (cos, sin) of pairs 2q, 2q + 1
                rotate(v[4 * q], v[4 * q + 1], cs[0], cs[1]);
                rotate(v[4 * q + 2], v[4 * q + 3], cs[2], cs[3]);
            }
        } else if constexpr (ROPE == kRopeSections) {
            // Table entry of pair j: f st + j (t section), base_h + y sh + j - sec0 (h),
            // base_w + x sw + j - sec1 (w).
            const int j0 = 16 * (wave & 3) + 8 * h;  // pairs of this lane within the head
            const int at_t = min(p.f, last_frame) * sec_len_t;  // tokens past the job (never stored) stay in the table
            const int at_h = e_base_h + p.y * sec_len_h - sec0;
            const int at_w = e_base_w + p.x * sec_len_w - sec1;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int j = j0 + i;
                const int entry = (j < sec0 ? at_t : (j < sec1 ? at_h : at_w)) + j;
                const f2 cs = *reinterpret_cast<const f2*>(rope_lds + 8 * entry);
                rotate(v[2 * i], v[2 * i + 1], cs[0], cs[1]);
            }
        }
        const __amdgpu_buffer_rsrc_t dst = make_rsrc(c_dst, c_dst_bytes);
        const uint32_t at = live && t0 + col < c_tokens ? c_lane + static_cast<uint32_t>(t0) * c_ts : kOutOfRange;
        if constexpr (OUT == RCH_DT_F32) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f4 out = {v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, out), dst, at + 16 * q, 0, 0);
            }
        } else if constexpr (OUT == RCH_DT_BF16) {
            bf8 x, y;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                x[i] = static_cast<__bf16>(v[i]);
                y[i] = static_cast<__bf16>(v[i + 8]);
            }
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, x), dst, at, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, y), dst, at + 16, 0, 0);
        } else {
            h8 x, y;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                x[i] = static_cast<_Float16>(v[i]);
                y[i] = static_cast<_Float16>(v[i + 8]);
            }
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, x), dst, at, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, y), dst, at + 16, 0, 0);
        }
    };

    // Software pipeline: the epilogue of unit u - 1 runs between the products of unit u, so the
    // matrix pipe keeps working while a wave rounds, rotates and stores (dense RoPE rows live in
    // per-unit LDS buffers and are used at once instead).
    constexpr bool kPipe = ROPE != kRopeDense;

    // Prologue: the first unit staged and converted, the consumer set up.
    stage_load();
    consumer_head(true);
    stage_store(0);
    __syncthreads();
    f16v prev = f16v{};  // accumulator of the unit whose epilogue is pending
    int prev_t0 = 0;
    GridPos prev_pos = pos;
    bool pending = false;
    for (int u = first; u < last; ++u) {
        const int buffer = (u - first) & 1;
        const bool more = u + 1 < last;
        if (more) {
            stager_advance();
            stage_load();  // issued before this unit's stores
        }
        // Products: 2 KS MFMAs on one accumulator, B fragments read from LDS three steps ahead.
        const uint8_t* fb = frags[buffer] + lane * 16;
        constexpr int kAhead = KS < 3 ? KS : 3;
        h8 ring[kAhead + 1];
#pragma unroll
        for (int s = 0; s < kAhead; ++s) ring[s] = *reinterpret_cast<const h8*>(fb + s * kFragPitch);
        f16v acc = f16v{};
        if constexpr (kPipe) {
            // The pending epilogue of unit u - 1 in pieces between the products (sched_barrier fences
            // keep each piece in place): RoPE table reads first, then the scale-and-bias roundings
            // and rotations spread over the steps, the casts and stores last.
            float v[16];
            f2 cs[8];
            const __amdgpu_buffer_rsrc_t dst = make_rsrc(c_dst, c_dst_bytes);
            const uint32_t at =
                pending && prev_t0 + col < c_tokens ? c_lane + static_cast<uint32_t>(prev_t0) * c_ts : kOutOfRange;
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                if (s + kAhead < KS) ring[(s + kAhead) % (kAhead + 1)] = *reinterpret_cast<const h8*>(fb + (s + kAhead) * kFragPitch);
                const h8 b = ring[s % (kAhead + 1)];
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(w_hi[s], b, acc, 0, 0, 0);
                if constexpr (ROPE == kRopeSections) {
                    if (s == 0) {
                        const int j0 = 16 * (wave & 3) + 8 * h;
                        const int at_t = min(prev_pos.f, last_frame) * sec_len_t;
                        const int at_h = e_base_h + prev_pos.y * sec_len_h - sec0;
                        const int at_w = e_base_w + prev_pos.x * sec_len_w - sec1;
#pragma unroll
                        for (int i = 0; i < 8; ++i) {
                            const int j = j0 + i;
                            const int entry = (j < sec0 ? at_t : (j < sec1 ? at_h : at_w)) + j;
                            cs[i] = *reinterpret_cast<const f2*>(rope_lds + 8 * entry);
                        }
                    }
                }
                // Elements [16 s / KS, 16 (s + 1) / KS) rounded; pairs completed by them rotated.
#pragma unroll
                for (int i = 16 * s / KS; i < 16 * (s + 1) / KS; ++i) {
                    v[i] = __builtin_fmaf(prev[i], unscale, bias[i]);
                    if constexpr (ROPE == kRopeSections) {
                        if (i & 1) rotate(v[i - 1], v[i], cs[i >> 1][0], cs[i >> 1][1]);
                    }
                }
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(w_lo[s], b, acc, 0, 0, 0);
                if (s == KS - 1) {
                    if constexpr (OUT == RCH_DT_F32) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const f4 out = {v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
                            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, out), dst, at + 16 * q, 0, 0);
                        }
                    } else if constexpr (OUT == RCH_DT_BF16) {
                        bf8 x, y;
#pragma unroll
                        for (int i = 0; i < 8; ++i) {
                            x[i] = static_cast<__bf16>(v[i]);
                            y[i] = static_cast<__bf16>(v[i + 8]);
                        }
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, x), dst, at, 0, 0);
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, y), dst, at + 16, 0, 0);
                    } else {
                        h8 x, y;
#pragma unroll
                        for (int i = 0; i < 8; ++i) {
                            x[i] = static_cast<_Float16>(v[i]);
                            y[i] = static_cast<_Float16>(v[i + 8]);
                        }
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, x), dst, at, 0, 0);
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, y), dst, at + 16, 0, 0);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                if (s + kAhead < KS) ring[(s + kAhead) % (kAhead + 1)] = *reinterpret_cast<const h8*>(fb + (s + kAhead) * kFragPitch);
                const h8 b = ring[s % (kAhead + 1)];
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(w_hi[s], b, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(w_lo[s], b, acc, 0, 0, 0);
            }
            epilogue(acc, c_t0, pos, buffer, true);
        }
        if (!more) {
            if constexpr (kPipe) epilogue(acc, c_t0, pos, 0, true);
            break;
        }
        // The next unit's fragments go to the other buffer: every wave finished reading it one
        // barrier ago.
        stage_store(buffer ^ 1);
        prev = acc;
        prev_t0 = c_t0;
        prev_pos = pos;
        pending = true;
        // Advance the consumer to the unit just staged.
        c_t0 += kStreamTokens;
        bool new_head = false, new_job = false;
        if (c_t0 >= c_tokens) {
            c_t0 = 0;
            new_head = true;
            if (++c_head == heads) {
                c_head = 0;
                ++c_member;
                c_job = members[2 * c_member + 1];
                new_job = true;
            }
        } else if constexpr (ROPE == kRopeSections) {
            pos.advance(kStreamTokens, grid_w, grid_h);
        }
        if (new_head) {
            // The pending epilogue needs this (job, head)'s slab: finish it before switching.
            if constexpr (kPipe) epilogue(prev, prev_t0, prev_pos, 0, true);
            pending = false;
            if (new_job) __syncthreads();  // every wave is done with the previous job's section rows
            consumer_head(new_job);
        }
        __syncthreads();
    }
}

// Kernel arguments: jobs, members (int32 [n_members + 1][2]: first unit and descriptor index of
// each job of the group, then (total units, 0)), bounds, n_members, heads, pack_base (added to
// every rch_job.pack_ptr).
typedef void (*StreamFn)(const rch_job*, const int32_t*, const int32_t*, int, int, int64_t);

template <int ROPE, int OUT>
StreamFn stream_ks(int ks, int* chosen) {
    if (ks <= 4) { *chosen = 4; return restore_stream_kernel<4, ROPE, OUT>; }
    if (ks <= 8) { *chosen = 8; return restore_stream_kernel<8, ROPE, OUT>; }
    if (ks <= 12) { *chosen = 12; return restore_stream_kernel<12, ROPE, OUT>; }
    if (ks <= 16) { *chosen = 16; return restore_stream_kernel<16, ROPE, OUT>; }
    *chosen = 0;
    return nullptr;
}

template <int ROPE>
StreamFn stream_out(int ks, int out_dtype, int* chosen) {
    switch (out_dtype) {
        case RCH_DT_F32: return stream_ks<ROPE, RCH_DT_F32>(ks, chosen);
        case RCH_DT_F16: return stream_ks<ROPE, RCH_DT_F16>(ks, chosen);
        case RCH_DT_BF16: return stream_ks<ROPE, RCH_DT_BF16>(ks, chosen);
        default: *chosen = 0; return nullptr;
    }
}

}  // namespace

// Defined in restore_stream.hip; rope is a StreamRope mode.  nullptr when no variant covers the
// rank steps.
StreamFn pick_stream_fp16x2(int ks, int rope, int out_dtype, int* chosen);

}  // namespace rch
