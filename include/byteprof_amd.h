/*
 * byteprof_amd.h — C ABI of libbyteprof_amd.so, the gfx950 (MI355X) kernels of the batch-1 decode hot path:
 * skinny weight-only matmul (bf16 / int8 weights, 1..64 activation rows), the int8 matrix-vector product, and the
 * fused multi-step mLSTM recurrence of the drafting path.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers (HBM) owned by the caller; the library never allocates, frees, retains or
 *     synchronises, and never reads device memory from the host, so every call can be captured in a HIP graph.
 *   - `stream` is a hipStream_t passed as void* (0 = the null stream). Work is enqueued on it and nothing else.
 *   - Matrices are row-major and dense: x [M, K], w [N, K], y [M, N] (leading dimension = the column count).
 *   - Return value: BP_OK (0) on success; a positive value is the hipError_t of the failed launch; a negative value
 *     is one of the BP_E_* codes below (checked before anything is enqueued).
 *   - Numerics: fp32 accumulation; the per-row int8 scale is applied to the fp32 sum; output rounded to nearest-even
 *     bf16; the K order of every sum depends only on (N, K, waves, split), never on M, so output row i does not
 *     change with the number of rows in the call (bitwise).
 *
 * The reference interfaces these replace are cited per function (paths relative to the byteprof repository).
 */
#ifndef BYTEPROF_AMD_H
#define BYTEPROF_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BP_OK 0
#define BP_E_INVALID_ARG (-1)    /* a null pointer, a negative size or an inconsistent shape */
#define BP_E_UNSUPPORTED (-2)    /* a tile configuration or dtype that no compiled kernel implements */
#define BP_E_WORKSPACE (-3)      /* split > 1 and the workspace is null or smaller than bp_skinny_workspace_bytes() */

/* Element type codes. */
#define BP_DT_BF16 0
#define BP_DT_F16 1
#define BP_DT_F32 2
#define BP_DT_I8 3

/* Library version (major * 10000 + minor * 100 + patch). */
int bp_version(void);

/* Short static description of a status code returned by any bp_* function (BP_* and hipError_t codes). */
const char* bp_status_string(int status);

/* Bytes of fp32 workspace a skinny call with this split needs: split * M * N * 4 when split > 1, else 0. */
size_t bp_skinny_workspace_bytes(int64_t M, int64_t N, int split);

/*
 * The skinny matmul of every row count on the matrix cores (v_mfma_f32_16x16x32_bf16), the path skinny_mm takes for
 * bf16 and int8 weights:
 *   y[M, N] (bf16) = x[M, K] (bf16) . w[N, K]^T, w bf16 (wkind 0) or int8 (wkind 1, times scale[N] of scale_dtype
 *   BP_DT_BF16 / F16 / F32 on the fp32 sum), 1 <= M <= 64 per call (M = 0 or N = 0: no-op; K = 0: zeros).
 * One load instruction reads a 128-byte segment of 8 consecutive weight rows (one full line per row); the
 * activations are the MFMA's B operand (8 activation rows per 16 columns, the other 8 columns carry the other half of
 * the segment's K slots). Tile configuration: rb = 8-row weight blocks per workgroup (1, 2, 4; 4 up to M = 16),
 * waves = wavefronts sharing the workgroup's K segments (1, 2, 4, 8; segment s to wave s % waves), split = K ranges
 * in separate workgroups whose fp32 partials are added in split order by a second kernel (workspace as for
 * bp_skinny_workspace_bytes), xstage: flags BP_XS_STAGE (each workgroup copies its activation rows and K range to
 * LDS first; up to M = 16 and bp_skinny_mf_stage_bytes() >= 0; else the activation operands are loaded with the
 * weights) and BP_XS_GENERAL (the general segment loop; without it, a launch whose waves have exactly 4, 8 or 16
 * segments each runs a straight-line kernel for that count); with BP_XS_STAGE at 9..16 rows, BP_XS_ROWS2 /
 * BP_XS_ROWS4 make the workgroup 2 / 4 row groups of rb blocks, each with its own `waves` waves, over one LDS copy of
 * the activation rows (the activation bytes per weight row fall 2 / 4x; up to 64 KiB of LDS,
 * bp_skinny_mf_stage_bytes_rows(); waves x groups <= 16; not with 16 segments a wave). The K order of every sum
 * depends only on (K, waves, split): output row i is bitwise independent of M (1..64), rb and xstage. K not a multiple of the 128-byte segment
 * (64 bf16 / 128 int8 elements), x, w not 16-byte aligned, or K >= 2^24 (the vector loads read the activations
 * through one buffer resource, under 2^31 bytes at 64 rows): an element-load variant with the same segments (rb 1,
 * 4 waves, xstage 0).
 * Replaces: byteprof/optim/skinny.py:36-90 (_skinny_kernel MODE 0 / 1, _split_reduce) and :111-133 (_launch) via
 *           skinny_mm (skinny.py:136-166) for every BM bucket (16, 32, 64); at M = 1 with int8 weights, the one-row
 *           int8 product byteprof/quant/triton_int8.py:16-47 (_gemv_int8, gemv_int8).
 */
#define BP_XS_STAGE 1
#define BP_XS_GENERAL 2
#define BP_XS_ROWS2 4
#define BP_XS_ROWS4 8
int bp_skinny_mf_supported(int wkind, int M, int rb, int waves, int xstage);
int bp_skinny_mf_k_segment(int wkind);
/* LDS bytes a launch with BP_XS_STAGE uses, or -1 when its activations do not fit (then the flag must be off). */
int64_t bp_skinny_mf_stage_bytes(int wkind, int64_t M, int64_t K, int split);
/* The same for a launch with BP_XS_STAGE and the row-group flags of xstage (their larger LDS limit). No counterpart in
 * the reference (its kernel stages nothing). */
int64_t bp_skinny_mf_stage_bytes_rows(int wkind, int64_t M, int64_t K, int split, int xstage);
int bp_skinny_mf(int wkind, const void* x, const void* w, const void* scale, int scale_dtype, void* y, int64_t M,
                 int64_t N, int64_t K, int rb, int waves, int split, int xstage, void* workspace,
                 size_t workspace_bytes, void* stream);
/* bp_skinny_mf stopped after the partial sums (split >= 2): workspace [split][M][N] fp32, unscaled for int8 (the
 * reducer applies the scale), e.g. for bp_decode_splitk_norm_residual_rows. */
int bp_skinny_mf_partials(int wkind, const void* x, const void* w, int64_t M, int64_t N, int64_t K, int rb,
                          int waves, int split, int xstage, void* workspace, size_t workspace_bytes, void* stream);
/* The gate|up projection with the SiLU product as the epilogue (split 1, 1 <= M <= 16): w [2 ffn, K] with row 2f the
 * gate row f and row 2f + 1 the up row f; out [M, ffn] = bf16(bf16(silu(bf16(g))) * bf16(u)) of the row sums, equal
 * bit for bit to bp_skinny_mf (same rb, waves, split 1) followed by bp_decode_silu_mul_rows (interleaved).
 * Replaces: the gate / up projections and act_fn(gate) * up of HF Olmo2MLP in the decode step that
 *           byteprof/optim/olmo.py:122-219 captures. */
int bp_skinny_mf_silu(int wkind, const void* x, const void* w, const void* scale, int scale_dtype, void* out,
                      int64_t M, int64_t ffn, int64_t K, int rb, int waves, int xstage, void* stream);

/*
 * bp_skinny_mf without a caller workspace and without allocating: the split-K partials go to a fixed device array
 * of bp_skinny_mf_static_bytes() bytes (8 MiB) inside the library, one per GPU, held until the process ends.
 * split x M x N x 4 must fit it (else BP_E_WORKSPACE before anything runs); calls that overlap on one GPU share the
 * array and race (order them on one stream). No counterpart in the reference (whose skinny_mm allocates the
 * workspace per call): for callers that cannot allocate device memory, such as code under HIP graph capture or
 * tight serving loops. Same outputs as bp_skinny_mf with the same plan, bit for bit.
 */
size_t bp_skinny_mf_static_bytes(void);
int bp_skinny_mf_static(int wkind, const void* x, const void* w, const void* scale, int scale_dtype, void* y,
                        int64_t M, int64_t N, int64_t K, int rb, int waves, int split, int xstage, void* stream);

/*
 * bp_skinny_mf with a transform of the activation rows first (split 1, K a multiple of the segment, 16-byte aligned
 * x and w, and the rows staged in LDS: M x K x 2 bytes <= 32 KiB, e.g. 8 rows of 2048 or one of 16384; the first
 * 2048 x waves elements pass through registers, the rest are loaded into LDS directly): the matmul reads
 *   BP_PRO_UNIT_RMS: bf16(x * (1 / sqrt(mean(x^2)))) per row (an all-zero row as is): a decode step's renormalised
 *                    input of the next linear;
 *   BP_PRO_NORM:     bf16(residual + bf16(gamma * (x * (1 / sqrt(mean(x^2) + eps))))) per row (residual NULL: the
 *                    plain norm), bit for bit bp_decode_norm_residual's output (its summation order), so that the
 *                    norm of a sublayer's output and the residual add run inside the next linear;
 * and when xout is not NULL the transformed rows [M, K] are written there (by one workgroup; an xout whose M x K
 * elements overlap those of x or of residual is refused with BP_E_INVALID_ARG before anything is enqueued). With gamma2 (BP_PRO_NORM only) the matmul reads bf16(gamma2 * (t * (1 / sqrt(mean(t^2) + eps))))
 * of those rows t instead (xout still receives t): a decoder's last post-feed-forward norm and its final norm in the
 * LM head's launch, bit for bit bp_decode_norm_residual followed by the BP_PRO_NORM launch. gamma, residual, xout
 * and gamma2 16-byte aligned. BP_PRO_NORM keeps gamma, the residual rows and gamma2 in LDS
 * beside the staged rows at one row, and at more rows while all of it fits 80 KiB (else it reads them from memory;
 * the same result). epilogue 0: y [M, N] = the plain product; 1: the gate|up SiLU product of bp_skinny_mf_silu,
 * y [M, N] with w [2 N, K] interleaved.
 * Replaces: RMSNorm / residual add before the next linear in the decode step (HF Olmo2DecoderLayer, post-attention
 *           and post-feed-forward norms) followed by the linear's skinny_mm call (byteprof/optim/olmo.py:164-215).
 */
#define BP_PRO_UNIT_RMS 1
#define BP_PRO_NORM 2
typedef struct BpPrologue {
  int32_t kind;          /* BP_PRO_UNIT_RMS or BP_PRO_NORM */
  float eps;             /* BP_PRO_NORM: added to the mean square inside the root */
  const void* gamma;     /* BP_PRO_NORM: bf16 [K] */
  const void* residual;  /* BP_PRO_NORM: bf16 [M, K], or NULL */
  void* xout;            /* bf16 [M, K], or NULL */
  const void* gamma2;    /* BP_PRO_NORM: bf16 [K]: a second norm of the transformed rows (no residual), or NULL */
} BpPrologue;
int bp_skinny_mf_pro(int wkind, const void* x, const void* w, const void* scale, int scale_dtype, void* y, int64_t M,
                     int64_t N, int64_t K, int rb, int waves, int epilogue, const BpPrologue* prologue, void* stream);

/*
 * The decode-step linear set in one launch of the skinny matrix-core kernel (M = 1): a grid over row blocks of a
 * list of linears ("items", in stage order), each workgroup owning 8 rb rows of one item.
 *   independent (dependent = 0): each item reads its own input x[K] -- the reference's set benchmark, where every
 *   linear is a separate skinny call (tools/skinny_bench.py:45-71);
 *   dependent (dependent = 1): an item may read a slice of an earlier stage's output instead (tag_in), optionally
 *   renormalised to unit RMS (bf16(v / sqrt(mean(v^2)))), as a decode step's linears wait for each other
 *   (byteprof/optim/olmo.py:122-219). A workgroup's weight loads (its whole tile when it fits 16 segments per wave)
 *   are issued before it waits, so the weights stream across stage boundaries. Outputs travel as 32-bit
 *   [generation tag : bf16] words (tag_out).
 * Every wait is bounded; a wait that gives up, or a tag_in item in an independent launch, sets scratch word 2 (the
 * launch still finishes; its results are invalid).
 * Every output equals bp_skinny_mf's at M = 1 with the same waves (split 1), bit for bit. K a multiple of the
 * 128-byte segment and at most 8192; weights 16-byte aligned. waves 2, 4 or 8.
 * bp_chain_plan checks the items and fills rb (rb_req 1, 2 or 4 for every item, or 0: per item, the most 8-row
 * blocks whose whole tile is in flight at once), first_wg and dep_wgs, and the lookup table
 * [ceil(workgroups / 256)] when given; it returns the workgroup count or a negative BP_E_* code.
 * bp_chain_run launches the planned items (device copies of the items and the table); dependent launches first
 * advance the generation in the scratch with a one-thread kernel. The scratch (bp_chain_scratch_bytes(stages),
 * zeroed once, kept between launches, not shared by overlapping launches) holds the generation, the per-stage
 * counters (they only grow) and the error word, so graph replays need no reset.
 * Replaces: the 113 stream-ordered skinny_mm calls of the set (independent: skinny_bench.py:45-71; dependent: the
 *           linears of one captured decode step, olmo.py:164-215).
 */
#define BP_CHAIN_RENORM 1
typedef struct BpChainItem {
  const void* x;           /* external input [K] bf16, 8-byte aligned, or NULL when the input is tag_in */
  const void* w;           /* weights [n, K], bf16 or int8 */
  const void* scale;       /* int8: per-row scale [n] (the launch's scale dtype) */
  void* y;                 /* plain output [n] bf16, or NULL */
  uint32_t* tag_out;       /* the output as tagged words [n] (dependent launches), or NULL */
  const uint32_t* tag_in;  /* the producer's tagged words from the input's first element (8-byte aligned), or NULL */
  int64_t n;
  int64_t K;
  int32_t first_wg;        /* set by bp_chain_plan */
  int32_t flags;           /* BP_CHAIN_RENORM */
  int32_t stage;           /* non-decreasing over the items */
  int32_t dep_stage;       /* the stage whose output tag_in points into */
  int32_t dep_wgs;         /* set by bp_chain_plan: workgroups of dep_stage (its counter's step per launch) */
  int32_t rb;              /* set by bp_chain_plan: 8-row blocks per workgroup */
} BpChainItem;
int bp_chain_supported(int wkind, int rb_req, int waves);
size_t bp_chain_scratch_bytes(int num_stages);
int bp_chain_plan(BpChainItem* items, int num_items, int wkind, int rb_req, int waves, int32_t* lut,
                  int lut_capacity);
int bp_chain_run(int wkind, int scale_dtype, const void* dev_items, const void* dev_lut, int num_items,
                 int total_wgs, int waves, void* scratch, int dependent, void* stream);

/*
 * int4 group-128 weights in the tile-major format of byteprof's skinny kernels:
 *   packed uint8 [ceil(N / R), K / 128, R, 64]: the R rows (tile_rows: 16, 32 or 64) of one row tile and one group of
 *   128 inputs form a contiguous R x 64-byte block; byte j of a row's group holds code j (low nibble) and code
 *   j + 64 (high nibble), codes 0..15; padding rows of the last tile are ignored;
 *   scale [K / 128, N] (scale_dtype BP_DT_BF16 / BP_DT_F16 / BP_DT_F32), zero [K / 128, N] fp16.
 * y[M, N] (bf16) = sum over groups g of scale[g, n] * sum_j (code - zero[g, n]) * x[m, 128 g + j], fp32; the codes,
 * zeros and activations enter the products exactly. 1 <= M <= 16; K a multiple of 128; x and packed 16-byte aligned.
 * waves: 1, 2, 4 or 8 (groups dealt to the waves); split: as for the other skinny kernels (the scale is applied per
 * group, so the reduce adds the partial sums as they are). The K order depends only on (K, waves, split) and on
 * which of two kernels runs: the matrix-core kernel (the activation rows as MFMA columns: nearly the same time at
 * any M) when N % 4 == 0, zero is 8-byte aligned, scale aligned to four of its elements and K < 2^24 (its
 * activations through one buffer resource); else a VALU kernel.
 * Replaces: byteprof/optim/skinny.py:46-63 (_skinny_kernel MODE 3) via skinny_mm (skinny.py:136-166).
 */
int bp_skinny_int4_config_supported(int mt, int tile_rows, int waves);
int bp_skinny_int4(const void* x, const void* packed, const void* scale, int scale_dtype, const void* zero, void* y,
                   int64_t M, int64_t N, int64_t K, int tile_rows, int waves, int split, void* workspace,
                   size_t workspace_bytes, void* stream);
/* bp_skinny_int4 of an interleaved gate|up weight ([2 ffn, K] packed: row 2f the gate row f, row 2f + 1 the up row
 * f) with the SiLU product as the epilogue: out [M, ffn] = bf16(bf16(silu(bf16(g))) * bf16(u)), equal bit for bit to
 * bp_skinny_int4 (same tile rows and waves, split 1) followed by bp_decode_silu_mul_rows (interleaved). The
 * matrix-core kernel only (ffn even, zero 8-byte aligned, scale aligned to four of its elements, K < 2^24), else
 * BP_E_UNSUPPORTED.
 * Replaces: the gate / up projections and act_fn(gate) * up of HF Olmo2MLP (with int4_wo weights) in the decode step
 *           that byteprof/optim/olmo.py:122-219 captures. */
int bp_skinny_int4_silu(const void* x, const void* packed, const void* scale, int scale_dtype, const void* zero,
                        void* out, int64_t M, int64_t ffn, int64_t K, int tile_rows, int waves, void* stream);
/* bp_skinny_int4 (epilogue 0: y [M, N]) or bp_skinny_int4_silu (epilogue 1: y [M, N] of an interleaved [2 N, K]
 * weight) with a prologue on the activation rows, as bp_skinny_mf_pro's: BP_PRO_NORM (residual add, xout, gamma,
 * an optional gamma2) or BP_PRO_UNIT_RMS; equal bit for bit to bp_decode_norm_residual_rows (or its unit-RMS form)
 * followed by the plain launch with the same tile rows and waves. M <= 8, split 1, bf16 scales and (2 M + 2) K x 2
 * bytes <= 64 KiB (the rows, gamma, the residual rows and gamma2 staged in LDS: K <= 8192 at one row, 2048 at up to
 * 7), else BP_E_UNSUPPORTED; xout may not overlap x or the residual rows (BP_E_INVALID_ARG).
 * Replaces: the RMSNorm / residual add before the next linear of HF Olmo2DecoderLayer (with int4_wo weights) in the
 *           decode step that byteprof/optim/olmo.py:122-219 captures. */
int bp_skinny_int4_pro(const void* x, const void* packed, const void* scale, int scale_dtype, const void* zero, void* y,
                       int64_t M, int64_t N, int64_t K, int tile_rows, int waves, int epilogue,
                       const BpPrologue* prologue, void* stream);

/*
 * Fixed-order reduction of split-K partial sums: y[M, N] = bf16(scale[n] * sum_{s < split} ws[s, M, N]);
 * scale may be null (bf16 weights). bp_skinny_mf and bp_skinny_int4 call it themselves when split > 1; it is
 * exported for callers that produce partial sums of their own (bp_skinny_mf_partials).
 * Replaces: byteprof/optim/skinny.py:84-90 (_split_reduce).
 */
int bp_splitk_reduce(const void* workspace, void* y, const void* scale, int scale_dtype,
                     int64_t M, int64_t N, int split, void* stream);

/*
 * Fused mLSTM recurrence over T positions from a read-only start state (batch 1).
 *   c [NH, DQ, DV], n [NH, DQ], m [NH]: start state, fp32, contiguous; never written.
 *   q, k [T, NH, DQ]; v [T, NH, DV]: io_dtype (BP_DT_BF16, BP_DT_F16 or BP_DT_F32); i, f [T, NH]: gate_dtype.
 *   h [>= T, NH, DV]: io_dtype, receives the cell outputs.
 *   nstart [NH, DQ], mstart [NH]: fp32, receive copies of the start n and m (for a later commit).
 *   str_*: element strides along T of q/k, v, i/f and h; the inner dimensions are contiguous.
 * Per position (f and i are pre-activations):
 *   m' = max(logsigmoid(f) + m, i); fa = exp(logsigmoid(f) + m - m'); ia = exp(i - m'); mv = exp(-m'),
 *   the three rounded to io_dtype; C <- fa C + ia k v^T; n <- fa n + ia k (fp32 state);
 *   h = (qs . io(C)) / (max(|qs . io(n)|, mv) + eps) with qs = q * qk_scale, stored as io_dtype.
 * bv: value columns per workgroup (4, 8 or 16); DQ a multiple of 64 up to 256, or 384 / 512 (workgroups of DQ or
 * DQ / 2 threads, whole 64-lane waves); other DQ: BP_E_UNSUPPORTED.
 * Replaces: byteprof/optim/draft_fused.py:27-40 (multistep_fw) and byteprof/optim/mlstm_multistep.py:21-86
 *           (_gates, multistep_fw_kernel).
 */
int bp_mlstm_multistep(const void* c, const void* n, const void* m,
                       const void* q, const void* k, const void* v, const void* i, const void* f,
                       void* h, void* nstart, void* mstart,
                       int T, int NH, int DQ, int DV,
                       int64_t str_t_qk, int64_t str_t_v, int64_t str_t_if, int64_t str_t_h,
                       int io_dtype, int gate_dtype, float qk_scale, float eps, int bv, void* stream);

/*
 * One step from the state (c [NH, DQ, DV], n [NH, DQ], m [NH], fp32, read only) into the caller's buffers: h [NH, DV]
 * (io_dtype) and the next state c_new, n_new, m_new (fp32, same shapes; must not overlap c, n, m), so each
 * position's state can go to a history slot. q, k [NH, DQ], v [NH, DV]: io_dtype; i, f [NH]: gate_dtype; the
 * arithmetic of one bp_mlstm_multistep position, and the state bp_mlstm_lazy_commit computes for L = 0; the same
 * DQ and bv rules.
 * Replaces: byteprof/optim/draft_core.py:114-141 (mlstm_step_into: the library's recurrent step kernel writing into
 *           given buffers).
 */
int bp_mlstm_step(const void* c, const void* n, const void* m, const void* q, const void* k, const void* v,
                  const void* i, const void* f, void* h, void* c_new, void* n_new, void* m_new, int NH, int DQ,
                  int DV, int io_dtype, int gate_dtype, float qk_scale, float eps, int bv, void* stream);

/*
 * Lazy commit of a verify round: the state after positions 0 .. L, with L = *length (an int64 in device memory, so
 * one captured graph serves every accepted length; clamped to the T positions that k, v, i, f hold), recomputed
 * from the start state with the same per-position update as bp_mlstm_multistep:
 *   c [NH, DQ, DV] fp32 holds the start C on entry and the committed C on return (in place);
 *   nstart [NH, DQ], mstart [NH] (the copies bp_mlstm_multistep made) -> n [NH, DQ], m [NH] (written).
 * k [T, NH, DQ], v [T, NH, DV]: io_dtype; i, f [T, NH]: gate_dtype; str_t_*: element strides along T.
 * Replaces: byteprof/optim/mlstm_multistep.py:89-134 (lazy_commit_kernel), draft_fused.py:43-56 (lazy_commit).
 */
int bp_mlstm_lazy_commit(void* c, void* n, void* m, const void* nstart, const void* mstart, const void* k,
                         const void* v, const void* i, const void* f, const void* length, int T, int NH, int DQ,
                         int DV, int64_t str_t_qk, int64_t str_t_v, int64_t str_t_if, int io_dtype, int gate_dtype,
                         int bv, void* stream);

/*
 * Accepted length of a verify pass, on the device: out[:S] <- tok[:S]; out[SMAX] <- the number of leading drafts
 * ids[1 + j] equal to tok[j] (j < S - 1). ids, tok, out: int64.
 * Replaces: byteprof/optim/mlstm_multistep.py:136-146 (accept_kernel), draft_fused.py:57-62 (accept).
 */
int bp_draft_accept(const void* ids, const void* tok, void* out, int S, int SMAX, void* stream);

/*
 * The end of a verify round of the token decode loop, on the device: bp_draft_accept's out[:S], out[SMAX] = L, then
 * the next round's inputs: ids[0] <- tok[L] (the token after the accepted prefix), *pos += L + 1. ids, tok, out,
 * pos: int64.
 * Replaces: the acceptance and set_state of byteprof/optim/olmo_draft.py (make_generate_draft's captured step:
 *           core.accepted_length_t, out_dev, set_state(tok[L], cp[0] + L + 1)).
 */
int bp_draft_verify_next(void* ids, const void* tok, void* out, int64_t* pos, int S, int SMAX, void* stream);

/*
 * cur <- hist[slot] for one layer's state, slot = *length (int64 in device memory, clamped to [0, slots)):
 * c_cur[i] = c_hist[slot * c_n + i] (i < c_n), likewise n (n_n <= c_n) and m (m_n <= c_n); fp32.
 * Replaces: byteprof/optim/draft_kernels.py (commit_kernel) via draft_core.py:92-111 (commit_state).
 */
int bp_draft_commit(const void* c_hist, void* c_cur, const void* n_hist, void* n_cur, const void* m_hist,
                    void* m_cur, const void* length, int64_t slots, int64_t c_n, int64_t n_n, int64_t m_n,
                    void* stream);

/*
 * The non-linear steps of one OLMo-2 decode step (batch 1), for a decode loop captured whole in one HIP graph: the
 * token id and the position are int64 values in device memory, read by the kernels, and the last step writes the
 * next token and advances the position, so that a replay needs no host value. bf16 tensors throughout; the
 * roundings are those of transformers' Olmo2ForCausalLM in bf16 with the eager attention (modeling_olmo2.py:
 * Olmo2RMSNorm, apply_rotary_pos_emb, eager_attention_forward, Olmo2MLP, Olmo2DecoderLayer).
 * Replaces: byteprof/optim/olmo.py:122-219 (make_generate_graph: the captured eager forward of the HF model, its
 * argmax and the in-graph update of the next step's inputs), with the linears done by bp_skinny_* launches.
 *
 * embed:          x[hidden] <- table[tok] (table [vocab, hidden]; tok clamped into range).
 * *_rows:         the same step for `rows` consecutive positions of a verify pass (row r of each [rows, ...]
 *                 operand at position *pos + r; the attention of row r covers positions 0 .. *pos + r, so the rows'
 *                 own cache entries, written by qk_rope_cache_rows before, take part causally); every row is
 *                 computed exactly as the one-row call at that position computes it.
 * qk_rope_cache:  qkv = [q | k | v] (3 * heads * head_dim); q, k RMSNorm'd over their whole length with their
 *                 weights, rotated by RoPE at *pos (inv_freq[head_dim / 2] fp32, cos / sin in fp32); q -> q_out;
 *                 k, v -> k_cache, v_cache [heads, max_len, head_dim] at row *pos (no write if *pos >= max_len);
 *                 head_dim a multiple of 8, qkv 16-byte aligned.
 * attention:      per head, positions 0 .. *pos: out = bf16(softmax_fp32(bf16(bf16(q . k) * scale)) as bf16 . v);
 *                 head_dim a multiple of 8 dividing 256, max_len <= 4096; caches 16-byte aligned.
 * rope_attention: qk_rope_cache and attention in one launch (one workgroup per head), equal bit for bit to the
 *                 two launches; qkv 16-byte aligned. rope_attention_rows: rows (<= 16, and rows x 3 x heads x
 *                 head_dim x 2 bytes of q|k|v under 2^31, else BP_E_UNSUPPORTED) consecutive positions
 *                 *pos .. *pos + rows - 1 (>= 0) in one launch (one workgroup per head and row), equal bit for bit
 *                 to qk_rope_cache_rows + attention_rows.
 * norm_residual:  out = bf16(residual + bf16(w * x * rsqrt(mean(x^2) + eps))), the mean square summed in one fixed
 *                 order (lane l of a 64-lane wave adds the squares of elements 256 j + 4 l + e in order, then an xor
 *                 butterfly over the lanes; bp_skinny_mf_pro uses the same); residual NULL: the plain norm;
 *                 out may alias residual. splitk_norm_residual_rows: x = the split-K reduce of a projection's
 *                 partials (workspace [split][rows][n] from bp_skinny_mf_partials, the int8 scale [n] applied,
 *                 NULL for bf16), equal bit for bit to bp_splitk_reduce + norm_residual_rows; n <= 16384.
 * silu_mul:       out[ffn] = bf16(bf16(silu(g)) * u), gate_up = [g | u] (2 * ffn); silu_mul_rows with
 *                 interleaved = 1 reads the pairs (gate_up[2f], gate_up[2f + 1]) instead.
 * argmax_next:    *tok = first index of the largest logit (NaN counts as largest); *pos += 1. Several workgroups
 *                 share the logits and the last to finish writes the result; `scratch` (8-byte aligned) holds
 *                 their partials (tagged with the call's generation, no fences), the generation, a counter and an
 *                 error word: bp_decode_argmax_scratch_bytes() bytes, zero before the first call, then reused as is
 *                 (each call leaves the counter at zero); calls sharing one scratch must not overlap. The error
 *                 word (u32 at index BP_ARGMAX_ERROR_WORD of a row's scratch) becomes 1 when the last workgroup
 *                 gave up waiting for a partial (a token written after that is not to be trusted); nothing in the
 *                 library clears it, so one read after a run covers every call of the run.
 * argmax_rows:    tok[r] = argmax of row r of logits [rows, vocab] (as argmax_next; no position update), with
 *                 bp_decode_argmax_rows_scratch_bytes(rows) bytes of scratch (8-byte aligned, zero before the
 *                 first call): BP_ARGMAX_ROW_WORDS u32 words per row, row r's error word at
 *                 r * BP_ARGMAX_ROW_WORDS + BP_ARGMAX_ERROR_WORD.
 */
int bp_decode_embed(const int64_t* tok, const void* table, void* x, int hidden, int64_t vocab, void* stream);
int bp_decode_embed_rows(const int64_t* tok, const void* table, void* x, int rows, int hidden, int64_t vocab,
                         void* stream);
int bp_decode_qk_rope_cache(const void* qkv, const void* q_norm_w, const void* k_norm_w, const float* inv_freq,
                            const int64_t* pos, void* q_out, void* k_cache, void* v_cache, int heads, int head_dim,
                            int max_len, float eps, void* stream);
int bp_decode_qk_rope_cache_rows(const void* qkv, const void* q_norm_w, const void* k_norm_w, const float* inv_freq,
                                 const int64_t* pos, void* q_out, void* k_cache, void* v_cache, int heads,
                                 int head_dim, int max_len, float eps, int rows, void* stream);
int bp_decode_attention(const void* q, const void* k_cache, const void* v_cache, const int64_t* pos, void* out,
                        int heads, int head_dim, int max_len, float scale, void* stream);
int bp_decode_attention_rows(const void* q, const void* k_cache, const void* v_cache, const int64_t* pos, void* out,
                             int heads, int head_dim, int max_len, float scale, int rows, void* stream);
int bp_decode_rope_attention(const void* qkv, const void* q_norm_w, const void* k_norm_w, const float* inv_freq,
                             const int64_t* pos, void* k_cache, void* v_cache, void* out, int heads, int head_dim,
                             int max_len, float eps, float scale, void* stream);
int bp_decode_rope_attention_rows(const void* qkv, const void* q_norm_w, const void* k_norm_w, const float* inv_freq,
                                  const int64_t* pos, void* k_cache, void* v_cache, void* out, int heads, int head_dim,
                                  int rows, int max_len, float eps, float scale, void* stream);
int bp_decode_splitk_norm_residual_rows(const float* workspace, int split, const void* scale, int scale_dtype,
                                        const void* weight, const void* residual, void* out, int n, float eps,
                                        int rows, void* stream);
int bp_decode_norm_residual(const void* x, const void* weight, const void* residual, void* out, int n, float eps,
                            void* stream);
int bp_decode_norm_residual_rows(const void* x, const void* weight, const void* residual, void* out, int n,
                                 float eps, int rows, void* stream);
int bp_decode_silu_mul(const void* gate_up, void* out, int ffn, void* stream);
int bp_decode_silu_mul_rows(const void* gate_up, void* out, int ffn, int rows, int interleaved, void* stream);
#define BP_ARGMAX_ROW_WORDS 132
#define BP_ARGMAX_ERROR_WORD 130
size_t bp_decode_argmax_scratch_bytes(void);
int bp_decode_argmax_next(const void* logits, int vocab, int64_t* tok, int64_t* pos, void* scratch, void* stream);
size_t bp_decode_argmax_rows_scratch_bytes(int rows);
int bp_decode_argmax_rows(const void* logits, int vocab, int rows, int64_t* tok, void* scratch, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BYTEPROF_AMD_H */
