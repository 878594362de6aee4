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
 * binds these symbols with ctypes (reelcache_amd/_lib.py lists every signature).  Each
 * declaration names the reference interface it replaces.
 */
#ifndef REELCACHE_HIP_H
#define REELCACHE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RCH_ABI_VERSION 12

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
#define RCH_JF_PIC_VEC4 8  /* pictures: every picture's base, the row and plane strides and grid_w are multiples
                              of 4 bytes, so 4 tokens (x % 4 == 0) of a cell row are one aligned 32-bit word */

/* Launch-group flags (rch_restore group_flags). */
#define RCH_GF_FAST 1      /* every job: uint8 codes with RCH_JF_SRC_VEC or pictures, RCH_JF_DST_VEC,
                              dst_bytes < 2**31, no device coefficient bound (bound_index < 0), and,
                              with RoPE, an interleaved pairs table under 2**31 bytes with an even row
                              stride; the group: head_dim % 32 == 0, channels == heads * head_dim */
#define RCH_GF_ROPE 2      /* with RCH_GF_FAST: every job of the group has RoPE (otherwise none has) */
#define RCH_GF_HEAD_PAIRS 4 /* with RCH_GF_FAST and an even head count: each work unit covers one
                               32-channel dim block of two adjacent heads (see rch_restore); only
                               for max_ksteps <= 12 (RCH_E_CONFIG otherwise).  Straight-line
                               variants cover max_ksteps <= 12 (fp16x2) or 16 (fp16, bf16); larger
                               ranks run the general kernel whatever the flags. */
#define RCH_GF_STREAM 16   /* with RCH_GF_FAST, fp16x2, uint8 code rows, head_dim 128, channels % 128 == 0,
                              max_ksteps <= 16, no other shape flag: the basis-stationary stream kernel.
                              Work units are (job, head, 32-token tile), job-major; tiles_dev holds
                              int32 [n_members + 1][2]: (first unit, job index) of each job of the group,
                              then (total units, 0); each job's pack_ptr points to its RCH_PACK_STREAM
                              slabs.  Its arithmetic folds the affine into the basis (exact fp16 codes),
                              so its output may differ from the other kernels' in the last bits. */
#define RCH_GF_DENSE_ROPE 32 /* with RCH_GF_STREAM and RCH_GF_ROPE: every job's table is dense (one row per
                               token).  Without it every job's table is separable and its section rows
                               (frames * sec_t + grid_h * sec_h + grid_w * sec_w pairs) number at most
                               RCH_STREAM_SECTION_PAIRS: the stream kernel stages them in LDS per job. */
#define RCH_STREAM_SECTION_PAIRS 2048
#define RCH_GF_SPLIT_RANK 8 /* with RCH_GF_FAST, uint8 code rows, not with RCH_GF_HEAD_PAIRS: the
                               straight-line kernel with 8-wave workgroups that split the rank
                               steps in two halves (max_ksteps up to 32); work units as without
                               flags.  Its fp32 sums add the halves' partial sums, so its output
                               may differ from the one-chain kernels in the last bit. */

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
    int64_t dst_ptr;         /* RCH_PACK_FRAGMENTS: ksteps * nblocks * 64 * frag bytes;
                                RCH_PACK_STREAM: nblocks slabs of RCH_STREAM_SLAB_BYTES(ksteps) */
    int64_t ksteps;          /* fragments: ceil(rank / 16); stream slabs: the stream kernel's rank steps,
                                exactly 4, 8, 12 or 16 and >= ceil(rank / 16) (other depths: no slab written) */
    int64_t nblocks;         /* fragments: 2 * ceil(channels / 64); stream slabs: channels / 32 */
    int64_t kind;            /* RCH_PACK_* */
    int64_t exp_ptr;         /* fragments: device int32 [nblocks], per 32-channel-block prescale exponents written here */
    int64_t scale_ptr, offset_ptr; /* stream slabs: the job's fp32 [rank] affine */
} rch_pack;                  /* 12 x int64 = 96 bytes */

/* Pack kinds.  RCH_PACK_FRAGMENTS: the basis rows as MFMA A-operand fragments (every kernel but
 * the stream kernel).  RCH_PACK_STREAM: one job's slabs for the stream kernel (RCH_GF_STREAM):
 * per 32-channel block, W = 2^e (s_k Q_kc) as fp16 hi and lo fragments ([ksteps] x 64 lanes x
 * 16 bytes each, hi first), the block's fp32 biases b_c = sum_k (o_k + 128 s_k) Q_kc (FP64 sum,
 * one rounding) in channel order, and the int32 exponent e. */
#define RCH_PACK_FRAGMENTS 0
#define RCH_PACK_STREAM 1
#define RCH_STREAM_SLAB_BYTES(ksteps) ((((int64_t)(ksteps)) * 2048 + 128 + 16 + 255) / 256 * 256)

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
 *              u = tile * ceil(channels / 32) + 32-channel block; with
 *              RCH_GF_HEAD_PAIRS, u = tile * (channels / 64) + unit of the tile
 *              (dim block u' / (heads / 2), heads 2 (u' % (heads / 2)) and the next).
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
 * Two launch groups of one call in one launch: a RoPE group and a plain group,
 * both RCH_GF_FAST | RCH_GF_HEAD_PAIRS with the same channels, head_dim,
 * source kinds (uint8 rows or pictures) and output dtype (f16 or bf16), each of
 * at most 12 rank steps, in fp16x2.  tiles_dev holds the RoPE group's
 * n_tiles0 tiles, then the plain group's n_tiles1; bounds_dev [grid + 1] splits
 * the concatenated head-pair units (as rch_restore with RCH_GF_HEAD_PAIRS) into
 * cost-balanced ranges.  Same values as one rch_restore per group; the grid
 * fills and drains once.  Replaces the per-group launches of _fused_group
 * (reelcache/restore_kernels.py:2025-2062) for a call's K and V groups.
 */
int rch_restore_pair(const rch_job* jobs_dev, int n_jobs, const int32_t* tiles_dev, int n_tiles0, int n_tiles1,
                     const int32_t* bounds_dev, int grid, int channels, int head_dim, int source_kind, int out_dtype,
                     int precision, int ksteps0, int ksteps1, const int32_t* scratch_dev, void* stream);

/*
 * Resident workgroups per CU of the rch_restore_pair kernel for these
 * arguments; 0 (and RCH_OK) when no pair kernel is compiled for them, in which
 * case the groups launch one by one.
 */
int rch_restore_pair_occupancy(int precision, int source_kind, int ksteps0, int ksteps1, int head_dim, int out_dtype,
                               int* blocks_per_cu);

/*
 * rch_basis_pack + rch_restore of one launch group that allocates nothing: the packed bases and
 * their block exponents live in a static device array of the library (RCH_NOALLOC_SCRATCH_BYTES
 * per device, held until the process ends) instead of memory the caller provides.  No
 * counterpart in the reference: it is for callers that cannot allocate device memory (code under
 * HIP-graph capture, tight serving loops, harnesses that forbid allocation).
 *   packs_host  host array of the group's packs (at most RCH_NOALLOC_MAX_PACKS); dst_ptr and
 *               exp_ptr are ignored: pack i goes to byte F_i = sum_{j<i} round_up(size_j, 256) of the
 *               fragment region, size = ksteps * nblocks * 64 * rch_fragment_bytes(precision) for
 *               RCH_PACK_FRAGMENTS and nblocks * RCH_STREAM_SLAB_BYTES(ksteps) for RCH_PACK_STREAM;
 *               fragment packs' block exponents go to word E_i = sum of nblocks over the earlier
 *               fragment packs.  Every pack's kind matches the group's kernel: stream slabs
 *               (RCH_GF_STREAM groups only) have ksteps equal to the stream variant that covers
 *               max_ksteps (4, 8, 12 or 16); fragment packs have ksteps = ceil(rank / 16).
 *               Anything else returns RCH_E_CONFIG before any launch.
 *   jobs_dev    as for rch_restore, except that a job of pack i carries pack_ptr = F_i (relative to
 *               the fragment region) and basis_exp_index = E_i, and bound_index = -1 (no device
 *               coefficient bounds: float sources in the fp16 modes need a host bound).
 * The other arguments are those of rch_restore.  Sizes beyond the array return RCH_E_CONFIG with
 * the sizes in the message.  Every call on a GPU shares its array, which keeps the last call's
 * contents: calls that overlap on one GPU (on different streams, or from several threads without
 * ordering) race; calls ordered on one stream do not.
 */
#define RCH_NOALLOC_SCRATCH_BYTES (32 << 20)
#define RCH_NOALLOC_WORD_BYTES 65536
#define RCH_NOALLOC_MAX_PACKS 8
int rch_restore_noalloc(const rch_pack* packs_host, int n_packs, const rch_job* jobs_dev, int n_jobs,
                        const int32_t* tiles_dev, int n_tiles, const int32_t* bounds_dev, int grid, int channels,
                        int head_dim, int source_kind, int out_dtype, int precision, int max_ksteps, int group_flags,
                        void* stream);

/*
 * Dense rows -> RoPE -> cast -> native store (DenseSource jobs).
 * Replaces _rope_store_kernel / _rope_store_group (reelcache/restore_kernels.py:1556-1585, :2124-2150).
 */
int rch_rope_store(const rch_job* jobs_dev, int n_jobs, const int32_t* tiles_dev, int n_tiles,
                   int channels, int head_dim, int out_dtype, void* stream);

/*
 * Staged comparison path (backend="staged"), one GEMM group at a time: the jobs of tiles_dev share
 * one basis and rank view, and their coefficient rows stack into one dense [rows, rank] work
 * matrix, job j's token t at row rows_dev[j] + t (int64 [n_jobs]; entries of other jobs unused).
 *
 * rch_staged_unpack writes that matrix: coefficients dequantized as float(q) * scale + offset with
 * two roundings (uint8 rows, pictures) or read as is (float sources), in the fp16 precision times
 * the job's power-of-two prescale 2^e (coef_exp, or the device bound's exponent when bound_index
 * >= 0: rch_coefficient_bound runs first), then rounded once to work_dtype (RCH_DT_F32 / F16 /
 * BF16).  tiles_dev: int32 [n_tiles][2] (job, first token) of 128-token tiles; work_stride in
 * elements, >= max_rank.  Replaces _unpack_kernel (reelcache/restore_kernels.py:1518-1554) as
 * _staged_group launches it (:2192-2230).
 *
 * The caller multiplies work @ Q[:rank] with the GPU BLAS library into an fp32 [rows, channels]
 * product (the reference's _staged_gemm, :2167-2189).
 *
 * rch_staged_store reads product row rows_dev[j] + t, multiplies by 2^-e (fp16), applies the job's
 * RoPE, casts and stores into the native slot.  Replaces _rope_store_kernel with PRESCALE as
 * _staged_group launches it (:1557-1585, :2244-2247).  precision: RCH_PREC_FP32, _FP16 or _BF16.
 */
int rch_staged_unpack(const rch_job* jobs_dev, int n_jobs, const int32_t* tiles_dev, int n_tiles,
                      const int64_t* rows_dev, void* work, int64_t work_stride, int max_rank, int source_kind,
                      int work_dtype, int precision, const int32_t* scratch_dev, void* stream);
int rch_staged_store(const rch_job* jobs_dev, int n_jobs, const int32_t* tiles_dev, int n_tiles,
                     const int64_t* rows_dev, const void* product, int64_t product_stride, int channels, int head_dim,
                     int out_dtype, int precision, const int32_t* scratch_dev, void* stream);

/* ------------------------------------------------------------------------------------------
 * Fit side (reelcache/gpu_fitting.py, reelcache/factorization.py, reelcache/node_packets.py).
 * ------------------------------------------------------------------------------------------ */

/*
 * One [rows, channels] source matrix X of a batched fit call, with its stored fp16 basis Q,
 * its fp32 coefficients P = X Q[:rank]^T and per-matrix device outputs.  Fields an entry point
 * does not use may be 0.  All pointers are device byte addresses, strides are in elements, and
 * every row has unit column stride.  X rows start 16-byte aligned (src_stride * element size
 * % 16 == 0) and channels % 8 == 0; the host pads other shapes with zero channels.
 */
typedef struct rch_fit_matrix {
    int64_t src_ptr;      /* X [rows, >= channels] */
    int64_t src_dtype;    /* RCH_DT_F32 / RCH_DT_F16 / RCH_DT_BF16 (one dtype per call) */
    int64_t rows;
    int64_t src_stride;
    int64_t basis_ptr;    /* fp16 Q [>= rank, channels] */
    int64_t basis_stride;
    int64_t rank;         /* 0: no basis (source energy only) */
    int64_t coef_ptr;     /* fp32 P [rows, >= rank]; coef_stride % 4 == 0, 16-byte aligned */
    int64_t coef_stride;
    int64_t gram_ptr;     /* fp32 G [channels, >= channels]; gram_stride % 4 == 0, 16-byte aligned */
    int64_t gram_stride;
    int64_t absmax_ptr;   /* uint32: fp32 bits of max|X| (zero-filled, then rch_fit_absmax) */
    int64_t extrema_ptr;  /* uint32 [2, rank]: ~key(min) then key(max) of each column of P, or 0 */
    int64_t energy_ptr;   /* float64 [2]: sum (X/s)^2 and sum ((X - P Q)/s)^2, s = max|X| */
    int64_t partial_ptr;  /* float64 [ceil(rows / 64), 2]: per-64-row partial energies */
    int64_t resid_ptr;    /* fp32 [rows, channels] (row stride = channels): X - P Q[:rank], or 0 */
} rch_fit_matrix;         /* 16 x int64 = 128 bytes */

int rch_fit_matrix_size(void);

/*
 * max|X| of each matrix as fp32 bits, combined with unsigned atomic max into *absmax_ptr
 * (zero-filled by the caller).  A non-finite element yields bits >= 0x7f800000.
 * Replaces `torch.maximum(tensor.amax().abs(), tensor.amin().abs())` and the finite scans of
 * project_onto_basis / measure_source_energy (reelcache/factorization.py:343-349, :708-712).
 */
int rch_fit_absmax(const rch_fit_matrix* mats_dev, int n_mats, int channels, int64_t max_rows, int src_dtype,
                   void* stream);

/*
 * Symmetric Gram G = X^T X of each matrix in fp32, both triangles written (exactly symmetric,
 * so (G + G^T) / 2 == G).  16-bit sources run on v_mfma_f32_32x32x16_{bf16,f16} (exact
 * products, fp32 accumulation), fp32 sources on v_mfma_f32_32x32x2f32.  Only the 128 x 128
 * tiles of the lower triangle are computed.
 * Replaces `torch.stack([mm(x.T, x) for x in sources])` + symmetrization of gram_bases and
 * _symmetric_gram (reelcache/gpu_fitting.py:286-289, reelcache/rank_method.py:634-638).
 */
int rch_fit_gram(const rch_fit_matrix* mats_dev, int n_mats, int channels, int src_dtype, void* stream);

/*
 * Coefficients P = X Q[:rank]^T of each matrix: exact products accumulated in FP64 on
 * v_mfma_f64_16x16x4f64, rounded once to fp32.  When extrema_ptr is set, also the per-column
 * min / max of P as order-preserving keys (unsigned atomic max, zero-filled by the caller).
 * Replaces `tensor.float() @ b32.T` of project_onto_basis (reelcache/factorization.py:384-392)
 * and the extrema of quantize_device (reelcache/node_packets.py:164).
 */
int rch_fit_project(const rch_fit_matrix* mats_dev, int n_mats, int channels, int64_t max_rows, int max_rank,
                    int src_dtype, void* stream);

/*
 * Direct residual and source energies of each matrix in FP64: sum (X / s)^2 and
 * sum ((X - P Q[:rank]) / s)^2 with s = max|X| read from *absmax_ptr (no scaling when s == 0),
 * the reconstruction accumulated in FP64 on v_mfma_f64_16x16x4f64.  Per-64-row partials go to
 * partial_ptr and are summed in a fixed order into energy_ptr (deterministic).  rank == 0
 * measures the source energy alone.  With resid_ptr set, also writes the residual matrix
 * fp32(X - P Q[:rank]) (the residual an inherited basis leaves for augmentation,
 * reelcache/rank_method.py:1347-1358).
 * Replaces the tiled residual guard of project_onto_basis (reelcache/factorization.py:398-419)
 * and measure_source_energy (reelcache/factorization.py:692-724).
 */
int rch_fit_residual(const rch_fit_matrix* mats_dev, int n_mats, int channels, int64_t max_rows, int src_dtype,
                     void* stream);

/*
 * Per-column extrema of an fp32 [rows, cols] matrix: keys[c] = ~key(min), keys[cols + c] =
 * key(max) (unsigned atomic max, zero-filled by the caller), key = order-preserving fp32 bits.
 * Replaces `torch.stack((coefficients.amin(0), coefficients.amax(0)))` of quantize_device
 * (reelcache/node_packets.py:164).
 */
int rch_column_extrema(const float* values_dev, int64_t rows, int cols, int64_t stride, uint32_t* keys_dev,
                       void* stream);

/*
 * 8-bit quantization: codes[r, c] = clamp(rint((double(v) - offset[c]) / scale[c]), 0, 255), 0 where
 * scale[c] == 0, in FP64 (round half to even).  Replaces the device arithmetic of quantize_device
 * (reelcache/node_packets.py:166-172) = _hevc.quantize_coefficients (reelcache/_hevc.py:465-472).
 */
int rch_quantize(const float* values_dev, int64_t rows, int cols, int64_t stride, const double* scale_dev,
                 const double* offset_dev, uint8_t* codes_dev, int64_t code_stride, void* stream);

/* One matrix of a batched quantization: fp32 values [rows, cols] -> uint8 codes. */
typedef struct rch_quantize_job {
    int64_t values_ptr;   /* fp32 [rows, >= cols], unit column stride */
    int64_t rows;
    int64_t cols;
    int64_t stride;       /* elements between rows of values */
    int64_t affine_ptr;   /* float64 [2, cols]: scale then offset */
    int64_t codes_ptr;    /* uint8 [rows, >= cols] */
    int64_t code_stride;
    int64_t reserved;
} rch_quantize_job;       /* 8 x int64 = 64 bytes */

/*
 * rch_quantize over a batch of matrices in one launch (grid: 64-row tiles x jobs), e.g. the
 * coefficients of every matrix of a chunk after projection.
 */
int rch_quantize_batched(const rch_quantize_job* jobs_dev, int n_jobs, int64_t max_rows, void* stream);

/* One block of seeded standard normals: fp32 dst[r * stride + c] for r < rows, c < cols. */
typedef struct rch_gauss_job {
    int64_t dst_ptr;
    int64_t rows;
    int64_t cols;
    int64_t stride;       /* elements between rows */
    int64_t seed;         /* 64-bit Philox-4x32-10 key */
    int64_t reserved[3];
} rch_gauss_job;          /* 8 x int64 = 64 bytes */

/*
 * Seeded Gaussian blocks of many matrices in one launch (grid: 1024-element groups x jobs):
 * element e = r * cols + c of a job is the (e % 4)-th normal of counter e / 4 (Philox-4x32-10
 * under the job's key, then Box-Muller), so a block's values depend only on its seed and shape.
 * max_elements = the largest rows * cols.  Replaces the per-matrix seeded torch generators of the
 * start blocks of gram / top-k directions and anchor sketches (reelcache/rank_method.py:479-484,
 * :591-631); the start columns only steer the solvers (every rank is verified on stored factors).
 */
int rch_fit_gaussian(const rch_gauss_job* jobs_dev, int n_jobs, int64_t max_elements, void* stream);

/*
 * Batched upper Cholesky factor and its inverse, in FP64: for each of n symmetric positive
 * definite k x k matrices A (row-major, contiguous, only the upper triangle read), R upper with
 * A = R^T R and x = R^{-1} (upper, zeros below).  info[b] = 0, or j + 1 when the leading minor of
 * order j + 1 is not positive definite (LAPACK's convention), x[b] is then the identity.
 * 1 <= k <= RCH_CHOLESKY_MAX_K (one workgroup per matrix, its upper triangle in LDS).
 * Replaces the torch.linalg.cholesky_ex + trsm_right_upper pair of each CholeskyQR step
 * (reelcache/rank_method.py:738-752, :676-685).
 */
#define RCH_CHOLESKY_MAX_K 128
int rch_cholesky_inverse(const double* a_dev, double* x_dev, int32_t* info_dev, int n, int k, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* REELCACHE_HIP_H */
