/*
 * reelcache_hip.h -- C ABI of the MI355X (gfx950) restore and fit kernels.
 *
 * Every entry point takes plain device addresses, sizes and a HIP stream
 * (hipStream_t passed as void*), enqueues its kernels on that stream and
 * returns 0, or a nonzero RCH_E_* status with a message readable through
 * rch_last_error() (thread-local).  Nothing here allocates device memory,
 * synchronizes the stream or changes process-wide state.
 *
 * The Python host (reelcache_amd/restore_kernels.py, reelcache_amd/gpu_fitting.py)
 * binds these symbols with ctypes; a reference-side binding is shown in
 * INTEGRATION.md.  Each declaration names the reference interface it replaces.
 */
#ifndef REELCACHE_HIP_H
#define REELCACHE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RCH_ABI_VERSION 2

/* Status codes (mapped to reelcache errors by the host). */
#define RCH_OK 0
#define RCH_E_CONFIG 1      /* ConfigurationError: invalid arguments */
#define RCH_E_UNSUPPORTED 2 /* UnsupportedError: combination not compiled / not available */
#define RCH_E_LAUNCH 3      /* a HIP launch or runtime call failed */

/* Precision codes: index into the reference's PRECISIONS tuple
 * (reelcache/restore_kernels.py:137). tf32 / tf32x3 are rejected on gfx950. */
#define RCH_PREC_FP32 0
#define RCH_PREC_TF32 1
#define RCH_PREC_TF32X3 2
#define RCH_PREC_FP16 3
#define RCH_PREC_FP16X2 4
#define RCH_PREC_BF16 5

/* Element dtypes. */
#define RCH_DT_F32 0
#define RCH_DT_F16 1
#define RCH_DT_BF16 2
#define RCH_DT_U8 3
#define RCH_DT_F64 4

/* Source kinds (reelcache/restore_kernels.py:1788-1794 _source_kind). */
#define RCH_SRC_FLOAT 0    /* CoefficientSource with float values */
#define RCH_SRC_U8 1       /* CoefficientSource with uint8 pixels + affine */
#define RCH_SRC_PICTURE 2  /* PictureSource (channel_tiles.v1 in place) */
#define RCH_SRC_DENSE 3    /* DenseSource ([N, C] rows) */

/* RoPE kinds (RopeTable sections / dense). */
#define RCH_ROPE_NONE 0
#define RCH_ROPE_SEPARABLE 1
#define RCH_ROPE_DENSE 2

/* Per-job flags (rch_job.flags). */
#define RCH_JF_SRC_VEC 1   /* coefficient rows: base and row stride 16-byte aligned, unit column stride */
#define RCH_JF_DST_VEC 2   /* destination: unit dim stride, 16-byte aligned base and token/head strides, head_dim % 16 == 0 */
#define RCH_JF_ROPE_VEC 4  /* RoPE tables: 16-byte aligned, row stride % 4 == 0, head_dim % 16 == 0 */

/* Launch-group flags (rch_restore group_flags). */
#define RCH_GF_FAST 1      /* every job: uint8 codes with RCH_JF_SRC_VEC or pictures, RCH_JF_DST_VEC,
                              dst_bytes < 2**31, no device coefficient bound (bound_index < 0), and,
                              with RoPE, an interleaved pairs table under 2**31 bytes with an even row
                              stride; the group: head_dim % 32 == 0, channels == heads * head_dim */
#define RCH_GF_ROPE 2      /* with RCH_GF_FAST: every job of the group has RoPE (otherwise none has) */

/*
 * One reconstruction job: one restored [N, C] matrix written into one native
 * cache slot.  Replaces one row of the reference's int64 descriptor table
 * (_FIELDS, reelcache/restore_kernels.py:160-172).  All pointers are device
 * byte addresses; strides are in elements.  64-bit throughout (no int32
 * in-job offset limit, cf. reelcache/restore_kernels.py:1806-1816).
 */
typedef struct rch_job {
    int64_t tokens;          /* N = frames * grid_h * grid_w */
    int64_t rank;            /* rank view (0 for dense sources) */
    int64_t frames, grid_h, grid_w;
    int64_t src_dtype;       /* RCH_DT_* of the coefficient / dense values */
    int64_t src_ptr;         /* coefficient [N, >=rank] or dense [N, C] base; picture base */
    int64_t src_row_stride, src_col_stride;
    int64_t scale_ptr, offset_ptr; /* fp32 [rank] affine (uint8 / picture sources) */
    int64_t coef_exp;        /* power-of-two prescale exponent of the coefficients (fp16 modes) */
    int64_t bound_index;     /* scratch word holding the device fp32 max|coef| (float sources without a host bound), or -1 */
    int64_t pack_ptr;        /* packed basis fragments (rch_basis_pack output) */
    int64_t pack_nblocks;    /* 32-channel blocks in the packed basis (even) */
    int64_t basis_exp_index; /* first scratch word of the pack's per-block exponents (written by rch_basis_pack) */
    int64_t dst_ptr;         /* byte address of (batch, token_offset, head 0, dim 0) */
    int64_t dst_token_stride, dst_head_stride, dst_dim_stride;
    int64_t rope;            /* RCH_ROPE_* */
    int64_t cos_ptr, sin_ptr, rope_row_stride; /* fp32 [rows, head_dim / 2] */
    int64_t row_t, row_h, row_w, sec_t, sec_h;
    int64_t pic_slots, pic_planes, pic_grid_cols, pic_plane_stride, pic_row_stride;
    int64_t pic_table_ptr;   /* device int64 [segments * frames] byte offsets from src_ptr */
    int64_t flags;           /* RCH_JF_* */
    int64_t pairs_ptr;       /* fp32 [rows, rope_row_stride, 2] interleaved (cos, sin), or 0 */
    int64_t pairs_bytes;     /* size of the pairs table in bytes */
    int64_t dst_bytes;       /* bytes from dst_ptr to one past the slot's last element */
    int64_t reserved;
} rch_job;                   /* 40 x int64 = 320 bytes */

/*
 * One basis to pack into MFMA A-operand fragments: rows Q[:rank] of a
 * [R, C] basis (unit column stride).  Fragment (s, nb, lane) holds 8 values
 * Q[k, c] for the 16-row step s and the 32-channel block nb.
 */
typedef struct rch_pack {
    int64_t src_ptr;         /* basis base address */
    int64_t src_dtype;       /* RCH_DT_F16 / RCH_DT_BF16 / RCH_DT_F32 */
    int64_t row_stride;      /* elements */
    int64_t rank;
    int64_t channels;
    int64_t dst_ptr;         /* packed fragments: ksteps * nblocks * 64 * frag bytes */
    int64_t ksteps;          /* ceil(rank / 16) */
    int64_t nblocks;         /* 2 * ceil(channels / 64) */
    int64_t reserved2;
    int64_t exp_ptr;         /* device int32 [nblocks]: per 32-channel-block prescale exponents written here */
    int64_t reserved[2];
} rch_pack;                  /* 12 x int64 = 96 bytes */

int rch_abi_version(void);
int rch_job_size(void);
int rch_pack_size(void);
const char* rch_last_error(void);
/* Size in bytes of one packed fragment for a precision (16 or 32). */
int rch_fragment_bytes(int precision);

/*
 * Pack bases into fragments for `precision` (fp16 for fp16/fp16x2, bf16 for
 * bf16, fp32 for fp32) and write each 32-channel block's prescale exponent
 * (non-zero only when a bf16/fp32 basis is packed as fp16: an exact power of
 * two bringing the block's max|Q| into (2**13, 2**14]).  The reference requires
 * the fp16 basis as is (reelcache/restore_kernels.py:1881-1882); a bf16 basis is
 * this build's superset.  Replaces the per-tile basis loads of
 * _fused_restore_kernel (reelcache/restore_kernels.py:1495-1496).
 * max_nblocks / max_ksteps = the largest nblocks / ksteps over the packs.
 */
int rch_basis_pack(const rch_pack* packs_dev, int n_packs, int64_t max_nblocks, int64_t max_ksteps, int precision,
                   void* stream);

/*
 * max|coefficient| per job for float sources in fp16 modes, written as fp32
 * bits with integer atomics into scratch[jobs[i].bound_index] (zero-filled by
 * the caller).  Replaces _bound_kernel (reelcache/restore_kernels.py:1587-1606).
 */
int rch_coefficient_bound(const rch_job* jobs_dev, int n_jobs, const int32_t* tiles_dev, int n_tiles,
                          int max_rank, int32_t* scratch_dev, void* stream);

/*
 * The fused restore: gather / dequantize coefficients, rank-view product on
 * MFMA, RoPE on interleaved pairs, cast and strided store into the native
 * cache.  One launch per launch group (jobs sharing source kind, channels,
 * head_dim and output dtype).
 *   tiles_dev  int32 [n_tiles, 2]: (job, first token) of every 128-token tile.
 *   bounds_dev int32 [grid + 1]: workgroup w processes work units
 *              [bounds[w'], bounds[w' + 1]) (w' = XCD-swizzled index), where unit
 *              u = tile * ceil(channels / 32) + 32-channel block.
 * max_ksteps = max ceil(rank / 16) over the group selects the compiled variant;
 * group_flags (RCH_GF_*) selects the straight-line variant for groups that qualify.
 * scratch_dev holds the basis exponents and device coefficient bounds the
 * descriptors index (basis_exp_index, bound_index).
 * Replaces _fused_restore_kernel / _fused_group / _two_pass_group
 * (reelcache/restore_kernels.py:1447-1515, :2025-2121).
 */
int rch_restore(const rch_job* jobs_dev, int n_jobs, const int32_t* tiles_dev, int n_tiles, const int32_t* bounds_dev,
                int grid, int channels, int head_dim, int source_kind, int out_dtype, int precision, int max_ksteps,
                int group_flags, const int32_t* scratch_dev, void* stream);

/*
 * Resident workgroups per CU of the rch_restore variant for these arguments
 * (sizes the persistent grid).  Replaces _channel_group's occupancy rule
 * (reelcache/restore_kernels.py:1979-1992).
 */
int rch_restore_occupancy(int precision, int source_kind, int max_ksteps, int head_dim, int out_dtype, int group_flags,
                          int* blocks_per_cu);

/*
 * Dense rows -> RoPE -> cast -> native store (DenseSource jobs).
 * Replaces _rope_store_kernel / _rope_store_group (reelcache/restore_kernels.py:1556-1585, :2124-2150).
 */
int rch_rope_store(const rch_job* jobs_dev, int n_jobs, const int32_t* tiles_dev, int n_tiles,
                   int channels, int head_dim, int out_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* REELCACHE_HIP_H */
