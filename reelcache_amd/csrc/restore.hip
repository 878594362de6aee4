// Restore entry points for MI355X (gfx950): basis packing, coefficient bounds, the dense
// RoPE store, and dispatch of the fused restore kernel (restore_kernel.h).
//
// Reference: reelcache/restore_kernels.py (_bound_kernel :1588-1606, _rope_store_kernel
// :1557-1585, _fused_group / _two_pass_group :2025-2121).
#include "restore_kernel.h"

namespace rch {
namespace {

// ---------------------------------------------------------------------------------------------
// Basis packing
// ---------------------------------------------------------------------------------------------

// One wave per (basis, 32-channel block): lane l holds channel block_channel(l % 32) and the
// rank slots of half l / 32.  Pass 1 reduces max|Q| over the block (fp16 fragments of a
// non-fp16 basis are prescaled by 2**e so that it lands in (2**13, 2**14]; one exponent per
// block, written to exps[block]); pass 2 writes the fragments of every 16-row step.
template <int PREC>
__global__ void __launch_bounds__(256) basis_pack_kernel(const rch_pack* __restrict__ packs) {
    const rch_pack& P = packs[blockIdx.y];
    const int64_t nb = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (nb >= P.nblocks) return;  // whole wave
    const int lane = threadIdx.x & 63, h = lane >> 5;
    const int64_t c = 32 * nb + block_channel(lane & 31);
    const int dtype = static_cast<int>(P.src_dtype);
    const bool scaled = (PREC == RCH_PREC_FP16 || PREC == RCH_PREC_FP16X2) && dtype != RCH_DT_F16;
    int e = 0;
    if (scaled) {
        float m = 0.0f;
        for (int64_t s = 0; s < P.ksteps; ++s) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int64_t k = 16 * s + k_slot<PREC>(h, j);
                if (k < P.rank && c < P.channels) m = fmaxf(m, fabsf(load_value(P.src_ptr, k * P.row_stride + c, dtype)));
            }
        }
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        e = prescale_exponent(m);
    }
    if (lane == 0) gout<int32_t>(P.exp_ptr)[nb] = e;
    const float pre = pow2f(e);
    for (int64_t s = 0; s < P.ksteps; ++s) {
        const int64_t q = (s * P.nblocks + nb) * 64 + lane;
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int64_t k = 16 * s + k_slot<PREC>(h, j);
            v[j] = (k < P.rank && c < P.channels) ? load_value(P.src_ptr, k * P.row_stride + c, dtype) : 0.0f;
        }
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
            h8 out;
#pragma unroll
            for (int j = 0; j < 8; ++j) out[j] = static_cast<_Float16>(v[j] * pre);
            gout<h8>(P.dst_ptr)[q] = out;
        }
    }
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

bool valid_out(int out_dtype) {
    return out_dtype == RCH_DT_F32 || out_dtype == RCH_DT_F16 || out_dtype == RCH_DT_BF16;
}

}  // namespace
}  // namespace rch

using namespace rch;

extern "C" {

int rch_fragment_bytes(int precision) { return precision == RCH_PREC_FP32 ? 32 : 16; }

int rch_basis_pack(const rch_pack* packs_dev, int n_packs, int64_t max_nblocks, int precision, void* stream) {
    if (!packs_dev || n_packs <= 0 || n_packs > 65535 || max_nblocks <= 0 || max_nblocks > 0x7fffffff)
        return fail(RCH_E_CONFIG, "rch_basis_pack: invalid arguments");
    const int64_t blocks = (max_nblocks + 3) / 4;
    const dim3 grid(static_cast<unsigned>(blocks), n_packs);
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

static int pick_variant(int precision, int source_kind, int max_ksteps, RestoreVariant* out) {
    switch (precision) {
        case RCH_PREC_FP32: *out = pick_restore_fp32(source_kind, max_ksteps); break;
        case RCH_PREC_FP16: *out = pick_restore_fp16(source_kind, max_ksteps); break;
        case RCH_PREC_FP16X2: *out = pick_restore_fp16x2(source_kind, max_ksteps); break;
        case RCH_PREC_BF16: *out = pick_restore_bf16(source_kind, max_ksteps); break;
        default: return fail(RCH_E_UNSUPPORTED, "precision %d has no matrix-core path on gfx950", precision);
    }
    if (!out->fn) return fail(RCH_E_CONFIG, "source kind %d is not a coefficient source", source_kind);
    return RCH_OK;
}

int rch_restore_occupancy(int precision, int source_kind, int max_ksteps, int* blocks_per_cu) {
    if (!blocks_per_cu || max_ksteps <= 0) return fail(RCH_E_CONFIG, "rch_restore_occupancy: invalid arguments");
    RestoreVariant variant;
    const int status = pick_variant(precision, source_kind, max_ksteps, &variant);
    if (status) return status;
    int blocks = 0;
    const hipError_t error = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &blocks, reinterpret_cast<const void*>(variant.fn), kThreads, 0);
    if (error != hipSuccess)
        return fail(RCH_E_LAUNCH, "rch_restore_occupancy: %s", hipGetErrorString(error));
    *blocks_per_cu = blocks;
    return RCH_OK;
}

int rch_restore(const rch_job* jobs_dev, int n_jobs, const int32_t* tiles_dev, int n_tiles, const int32_t* bounds_dev,
                int grid, int channels, int head_dim, int source_kind, int out_dtype, int precision, int max_ksteps,
                const int32_t* scratch_dev, void* stream) {
    if (!jobs_dev || !tiles_dev || !bounds_dev || !scratch_dev || n_jobs <= 0 || n_tiles <= 0 || grid <= 0 || channels <= 0 ||
        head_dim <= 0 || head_dim % 2 || max_ksteps <= 0 ||
        static_cast<int64_t>(n_tiles) * ((channels + 31) / 32) > 0x7fffffff)
        return fail(RCH_E_CONFIG, "rch_restore: invalid launch arguments");
    if (!valid_out(out_dtype)) return fail(RCH_E_CONFIG, "rch_restore: output dtype must be f32, f16 or bf16");
    RestoreVariant variant;
    const int status = pick_variant(precision, source_kind, max_ksteps, &variant);
    if (status) return status;
    const int nk = variant.chunked ? (max_ksteps + variant.ks - 1) / variant.ks : 1;
    hipLaunchKernelGGL(variant.fn, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, as_stream(stream), jobs_dev,
                       tiles_dev, bounds_dev, scratch_dev, nk, channels, head_dim, out_dtype);
    return check_launch("rch_restore");
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

}  // extern "C"
