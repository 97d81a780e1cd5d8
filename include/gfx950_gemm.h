/*
 * gfx950_gemm.h -- C ABI of the MI355X (gfx950) NT GEMM library.
 *
 * C[M,N] = A[M,K] . B[K,N] where both operands are K-contiguous in memory
 * ("NT": A is M rows of K values, B is N rows of K values).  Three operand
 * types: FP16/BF16 (a16w16), BF8 = fp8 e5m2 with optional per-tensor fp32
 * scales (a8w8), and MXFP4 = e2m1 packed two per byte with one E8M0 scale per
 * 32 K-values (a4w4).  Three tile schedules: data-parallel (one 256x256 tile per
 * workgroup), stream-K (persistent workgroups over (tile, K-stage) work with
 * a K-ordered fp32 fixup; bit-identical to data-parallel) and split-K (for
 * grids of fewer tiles than half the CUs: each tile's K range is cut into
 * segments computed in parallel and their fp32 partials are summed in a fixed
 * order by a second kernel; deterministic, within rounding of data-parallel).
 *
 * Every entry point takes raw device pointers, sizes and strides in ELEMENTS
 * (bytes for the uint8 MXFP4 operands and scales), launches asynchronously on
 * `stream` (a hipStream_t; NULL = default stream) and returns a status code.
 * Nothing is synchronised and nothing is allocated: the stream-K / split-K workspace is
 * owned by the caller (size from g9_workspace_size, zeroed once with
 * g9_workspace_init before first use, and not shared by launches that may run
 * concurrently).
 *
 * The per-dtype entry points replace the launch wrappers of the reference's
 * Gluon kernels (argument order a, b, c, M, N, K, stride_am, stride_ak,
 * stride_bk, stride_bn, stride_cm, stride_cn as in their kernel launches).
 */
#ifndef GFX950_GEMM_H
#define GFX950_GEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
enum {
  G9_OK = 0,
  G9_ERR_SHAPE = 1,     /* non-positive or unsupported M/N/K (K granularity: see each entry point) */
  G9_ERR_LAYOUT = 2,    /* K stride != 1, N stride of C != 1, operand rows not 16-byte aligned */
  G9_ERR_DTYPE = 3,     /* unsupported element / output type */
  G9_ERR_SCHEDULE = 4,  /* unknown schedule or wave count */
  G9_ERR_WORKSPACE = 5, /* stream-K / split-K workspace missing or too small */
  G9_ERR_HIP = 6,       /* the HIP runtime rejected the launch */
  G9_ERR_SCRATCH = 7,   /* g9_gemm_a16w16_noalloc: the call needs more than its static scratch buffer */
  G9_ERR_PLAN = 8       /* g9_plan_launch: plan not made by g9_plan_*, or made on another device */
};

/* Element / output types.  G9_FP4P is MXFP4 with preshuffled scales (the
 * operand type of g9_gemm_a4w4_preshuffled) and G9_FP4K MXFP4 with K-major
 * scales (g9_gemm_a4w4 given K-major scale views), both for g9_kernel_name
 * and g9_workspace_size. */
enum { G9_F16 = 0, G9_BF16 = 1, G9_BF8 = 2, G9_FP4 = 3, G9_FP4P = 4, G9_FP4K = 5 };

/* Tile schedules.  G9_SCHED_SPLITK has no counterpart in the reference: it is
 * for callers whose grids leave most CUs idle (few-row GEMMs, one GPU's
 * shard of a sharded GEMM).  G9_SCHED_SK_HALF is stream-K over 256 x 128
 * tiles (a16w16 only, 4 waves; G9_ERR_SCHEDULE otherwise), bit-identical to
 * data-parallel like G9_SCHED_SK, for grids with fewer 256 x 256 tiles than
 * CUs; no counterpart in the reference either. */
enum { G9_SCHED_DP = 0, G9_SCHED_SK = 1, G9_SCHED_SPLITK = 2, G9_SCHED_SK_HALF = 3 };

/*
 * a16w16: FP16 or BF16 (`dtype` = G9_F16 / G9_BF16) in and out, fp32 accumulate.
 * Replaces the launch in kernels/gemm/intra_wave/a16w16/v9_beyond_hotloop/matmul_kernel.py:390-424
 * (4-wave, `waves` = 4) and the missing 8-wave kernel bound by
 * kernels/gemm/inter_wave/a16w16/bench.py:48 (`waves` = 8).
 * K must be a multiple of 8 (16 bytes); the reference needs a multiple of
 * 128.  When K is not a multiple of 64 the first K stage is partial: its
 * loads of the missing leading chunks read zeros (operand row strides then
 * below 2^24 bytes).
 */
int g9_gemm_a16w16(const void* a, const void* b, void* c, int64_t M, int64_t N, int64_t K,
                   int64_t stride_am, int64_t stride_ak, int64_t stride_bk, int64_t stride_bn,
                   int64_t stride_cm, int64_t stride_cn, int dtype, int schedule, int waves,
                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * Allocation-free variant of g9_gemm_a16w16, for callers that cannot
 * allocate device memory or own a workspace (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  No counterpart in
 * the reference.  Same arguments, kernels and results as g9_gemm_a16w16
 * without the workspace: the stream-K and split-K partials live in a static
 * device array of the library (one per GPU, held until the process ends) of
 * G9_NOALLOC_MAX_TILES fp32 partial tiles of 256 x 256, or twice as many of
 * 256 x 128 (64 MiB), plus a header and flag words.  A call that needs more
 * (stream-K on more tiles, split-K with more segment tiles) returns
 * G9_ERR_SCRATCH; data-parallel needs none.
 * The call allocates nothing: a stream-K call first clears the array's flag
 * and error words with a fill kernel on `stream` (no memset), split-K writes
 * every partial it reads.  Calls share their GPU's array, so calls that may
 * overlap on one GPU (other streams, other host threads) race and must be
 * ordered by the caller.  A stream-K flag wait that times out leaves a wrong
 * output; g9_noalloc_error reports it.
 */
#define G9_NOALLOC_MAX_TILES 256
int g9_gemm_a16w16_noalloc(const void* a, const void* b, void* c, int64_t M, int64_t N, int64_t K,
                           int64_t stride_am, int64_t stride_ak, int64_t stride_bk, int64_t stride_bn,
                           int64_t stride_cm, int64_t stride_cn, int dtype, int schedule, int waves,
                           void* stream);

/*
 * Error word of the static array of g9_gemm_a16w16_noalloc on the device of
 * `stream`, copied to *error after synchronising `stream`: 1 when a flag wait
 * of the last stream-K call there timed out (that call's output is wrong),
 * else 0.  Each stream-K call clears it first, so read it before the next
 * one.  For the same callers as g9_gemm_a16w16_noalloc; allocates nothing.
 * No counterpart in the reference.
 */
int g9_noalloc_error(void* stream, int* error);

/*
 * a8w8: BF8 (fp8 e5m2) in, fp32 accumulate, C = (A.B) * a_scale[0] * b_scale[0]
 * written as `out_dtype` (G9_F16, the reference default, or G9_BF16).  The scale
 * pointers are device fp32 scalars; NULL means 1.0.
 * Replaces kernels/gemm/intra_wave/a8w8/matmul_kernel.py:437-470 (4-wave) and
 * kernels/gemm/inter_wave/a8w8/matmul_kernel.py:343-388 (8-wave).
 * K must be a multiple of 16 (16 bytes); a partial first stage when it is not
 * a multiple of 128, as for a16w16.
 */
int g9_gemm_a8w8(const void* a, const void* b, void* c, int64_t M, int64_t N, int64_t K,
                 int64_t stride_am, int64_t stride_ak, int64_t stride_bk, int64_t stride_bn,
                 int64_t stride_cm, int64_t stride_cn, const float* a_scale, const float* b_scale,
                 int out_dtype, int schedule, int waves, void* workspace, size_t workspace_bytes,
                 void* stream);

/*
 * a4w4: MXFP4.  a is M x K/2 bytes, b is N x K/2 bytes (two e2m1 values per
 * byte, low nibble = even k); a_scales is M x K/32 and b_scales N x K/32 E8M0
 * bytes (2^(x-127)).  K is the logical (unpacked) depth, a multiple of 256.
 * Strides are in bytes.  Output `out_dtype` (G9_BF16, the reference default,
 * or G9_F16).  The scales are row-major (stride_ask = stride_bsk = 1, row
 * strides multiples of 4), or both K-major (stride_asm = stride_bsn = 1,
 * group strides multiples of 4 of at least M and N bytes: the transposed
 * (K/32, M) storage the reference bench passes as its scale views), which the
 * 4-wave kernels read as they are (G9_ERR_SCHEDULE with `waves` = 8).
 * Replaces kernels/gemm/intra_wave/a4w4/v1_sliceMN/matmul_kernel.py:696-742 (4-wave)
 * and kernels/gemm/inter_wave/a4w4/v2_mfma32x32x64/matmul_kernel.py:614-668 (8-wave).
 */
int g9_gemm_a4w4(const void* a, const void* b, void* c, const void* a_scales, const void* b_scales,
                 int64_t M, int64_t N, int64_t K, int64_t stride_am, int64_t stride_ak,
                 int64_t stride_bn, int64_t stride_bk, int64_t stride_cm, int64_t stride_cn,
                 int64_t stride_asm, int64_t stride_ask, int64_t stride_bsn, int64_t stride_bsk,
                 int out_dtype, int schedule, int waves, void* workspace, size_t workspace_bytes,
                 void* stream);

/*
 * a4w4 with preshuffled E8M0 scales: the operands, output and results of
 * g9_gemm_a4w4 (bit-identical for the same scale values), with each operand's
 * scales in the kernel's read order instead of row-major.  Scales of stages
 * 4c..4c+3 (K values 1024c..1024c+1023) form chunk c, and row r of chunk c is
 * the 32 bytes at scales + c * stride_asc + 32 * r, whose byte 8j + 2s + h holds
 * the E8M0 scale of K group 32c + 8s + 4h + g with g = j ^ ((r >> 2) & 3)
 * (j, s in 0..3, h in 0..1); groups past K/32 may hold anything.  quant.preshuffle_e8m0 builds this
 * layout (stride = 32 * rows); the scales are 16-byte aligned, stride_asc and
 * stride_bsc multiples of 16 of at least 32 * M and 32 * N bytes (ignored when
 * K <= 1024: one chunk).  Each lane
 * then reads its scales of four stages with one LDS read and the scale DMAs
 * move contiguous KiB.  Data-parallel schedule, 4 waves.  No counterpart in the
 * reference: its roadmap lists preshuffled scales (its ROADMAP.md,
 * "4-bit + Scales", "Document preshuffling").
 */
int g9_gemm_a4w4_preshuffled(const void* a, const void* b, void* c, const void* a_scales, const void* b_scales,
                             int64_t M, int64_t N, int64_t K, int64_t stride_am, int64_t stride_ak,
                             int64_t stride_bn, int64_t stride_bk, int64_t stride_cm, int64_t stride_cn,
                             int64_t stride_asc, int64_t stride_bsc, int out_dtype, int schedule, int waves,
                             void* workspace, size_t workspace_bytes, void* stream);

/*
 * Prepared launches.  g9_plan_<op> takes the arguments of g9_gemm_<op>
 * without the stream, validates them and resolves the kernel, grid and
 * parameter block (and split-K's reduction) into *plan, returning the status
 * g9_gemm_<op> would return, without enqueueing anything.  g9_plan_launch
 * then only enqueues the plan on `stream`, which must belong to the device
 * that was current when the plan was made (G9_ERR_PLAN otherwise); a
 * stream-K plan takes a fresh flag epoch at each launch.  Each launch of a
 * plan is the launch g9_gemm_<op> makes with the same arguments (same
 * kernels, bit-identical results).  A plan is plain data (copyable, no
 * destructor, nothing allocated); it holds the operand and workspace
 * pointers, which must stay valid, and launches that share a workspace must
 * be ordered, as for g9_gemm_<op>.
 * Replaces the reference's prepared launches (scripts/prepared_kernel.py:53-138,
 * used by scripts/benchmark_prepared.py:135-271), which bind each rotating
 * argument set once so a timing loop enters the compiled launcher directly.
 */
#define G9_PLAN_BYTES 512
typedef struct g9_plan {
  uint64_t opaque[G9_PLAN_BYTES / 8];
} g9_plan;

int g9_plan_a16w16(g9_plan* plan, const void* a, const void* b, void* c, int64_t M, int64_t N, int64_t K,
                   int64_t stride_am, int64_t stride_ak, int64_t stride_bk, int64_t stride_bn,
                   int64_t stride_cm, int64_t stride_cn, int dtype, int schedule, int waves,
                   void* workspace, size_t workspace_bytes);
int g9_plan_a8w8(g9_plan* plan, const void* a, const void* b, void* c, int64_t M, int64_t N, int64_t K,
                 int64_t stride_am, int64_t stride_ak, int64_t stride_bk, int64_t stride_bn,
                 int64_t stride_cm, int64_t stride_cn, const float* a_scale, const float* b_scale,
                 int out_dtype, int schedule, int waves, void* workspace, size_t workspace_bytes);
int g9_plan_a4w4(g9_plan* plan, const void* a, const void* b, void* c, const void* a_scales, const void* b_scales,
                 int64_t M, int64_t N, int64_t K, int64_t stride_am, int64_t stride_ak,
                 int64_t stride_bn, int64_t stride_bk, int64_t stride_cm, int64_t stride_cn,
                 int64_t stride_asm, int64_t stride_ask, int64_t stride_bsn, int64_t stride_bsk,
                 int out_dtype, int schedule, int waves, void* workspace, size_t workspace_bytes);
int g9_plan_a4w4_preshuffled(g9_plan* plan, const void* a, const void* b, void* c, const void* a_scales,
                             const void* b_scales, int64_t M, int64_t N, int64_t K, int64_t stride_am,
                             int64_t stride_ak, int64_t stride_bn, int64_t stride_bk, int64_t stride_cm,
                             int64_t stride_cn, int64_t stride_asc, int64_t stride_bsc, int out_dtype,
                             int schedule, int waves, void* workspace, size_t workspace_bytes);
int g9_plan_launch(const g9_plan* plan, void* stream);

/*
 * Grouped ("MoE") GEMMs over E experts, 4-wave, data-parallel tiles.  The
 * rows of A (tokens, T in total) are sorted by expert: expert e owns rows
 * [expert_offsets[e], expert_offsets[e+1]) of A and of C and multiplies them
 * by its own B_e, the N x K operand stride_be bytes after B_(e-1) (rows
 * stride_bn apart, K-contiguous).  expert_offsets is a device array of E + 1
 * int32 prefix sums (offsets[0] = 0, offsets[E] <= T); rows of C outside every
 * expert's range are not written, offsets are clamped to [0, T] (so no table
 * makes the kernel access memory outside A, C and the E experts' B), and an
 * expert with no rows costs nothing.  No counterpart in the reference: its
 * roadmap plans an MXFP4 MoE kernel (its ROADMAP.md, "4-bit + Scales").
 *
 * g9_moe_a16w16: FP16 / BF16 (`dtype`), strides in elements except stride_be
 * (bytes); K a multiple of 64.
 */
int g9_moe_a16w16(const void* a, const void* b, void* c, const int32_t* expert_offsets, int64_t T,
                  int64_t N, int64_t K, int64_t E, int64_t stride_am, int64_t stride_bn, int64_t stride_be,
                  int64_t stride_cm, int dtype, void* stream);

/*
 * g9_moe_a8w8: BF8 (fp8 e5m2) as g9_gemm_a8w8 (strides in bytes): C rows of
 * expert e = (A . B_e^T) * a_scale[0] * b_scales[e], with a_scale one device
 * fp32 value and b_scales E of them (either NULL = 1.0); `out_dtype` G9_BF16
 * or G9_F16.  K a multiple of 128.
 */
int g9_moe_a8w8(const void* a, const void* b, void* c, const int32_t* expert_offsets, const float* a_scale,
                const float* b_scales, int64_t T, int64_t N, int64_t K, int64_t E, int64_t stride_am,
                int64_t stride_bn, int64_t stride_be, int64_t stride_cm, int out_dtype, void* stream);

/*
 * g9_moe_a4w4: MXFP4 as g9_gemm_a4w4 (strides in bytes); expert e's weights are
 * b + e * stride_be (N x K/2 bytes) and its scales b_scales + e * stride_bse
 * (N x K/32 bytes); `out_dtype` G9_BF16 or G9_F16.  K a multiple of 256.
 */
int g9_moe_a4w4(const void* a, const void* b, void* c, const void* a_scales, const void* b_scales,
                const int32_t* expert_offsets, int64_t T, int64_t N, int64_t K, int64_t E, int64_t stride_am,
                int64_t stride_bn, int64_t stride_be, int64_t stride_asm, int64_t stride_bsn,
                int64_t stride_bse, int64_t stride_cm, int out_dtype, void* stream);

/* Name of the grouped kernel g9_moe_* launches for (dtype, out_dtype), or NULL. */
const char* g9_moe_kernel_name(int dtype, int out_dtype);

/*
 * Bytes of workspace a call with these arguments needs (0 for the
 * data-parallel schedule, and for split-K when it runs as data-parallel).
 * `dtype` is the operand type.  Split-K's size depends on the current
 * device's CU count.  No counterpart in the reference (it has neither
 * stream-K nor split-K).
 */
size_t g9_workspace_size(int dtype, int64_t M, int64_t N, int64_t K, int schedule, int waves);

/*
 * Zeroes the flag and error words of a stream-K workspace on `stream`.  Call
 * once after allocating it.  No counterpart in the reference.
 */
int g9_workspace_init(void* workspace, size_t workspace_bytes, void* stream);

/*
 * Copies the workspace error word to *error (1 = a stream-K flag wait timed out
 * and the output is invalid) after synchronising `stream`.  No counterpart in
 * the reference.
 */
int g9_workspace_error(const void* workspace, size_t workspace_bytes, void* stream, int* error);

/*
 * Registers `host_flag`, an int in host memory the device can write (pinned:
 * hipHostMalloc), with a stream-K workspace: a launch whose flag wait times
 * out then also stores 1 there, so the caller learns of it without
 * synchronising (for instance by reading it before each launch).  Enqueued on
 * `stream` after g9_workspace_init, which clears the registration; NULL
 * removes it.  No counterpart in the reference.
 */
int g9_workspace_watch(void* workspace, size_t workspace_bytes, int* host_flag, void* stream);

/*
 * Polls a stream-K flag wait makes before it gives up, sets the error word
 * and carries on with whatever partial the workspace holds (0 restores the
 * default, 2^26, seconds of waiting).  Returns the previous value.  For tests
 * of the timeout path: a tiny limit makes waits time out while every
 * workgroup still exits normally.  Applies to launches made after the call.
 */
uint32_t g9_set_streamk_spin_limit(uint32_t polls);

/*
 * Byte transpose on `stream`: dst (cols x rows, row stride dst_ld bytes) =
 * src (rows x cols, row stride src_ld bytes) transposed.  The drop-in a4w4
 * wrapper repacks K-major E8M0 scale views, (K/32, M) storage seen as
 * (M, K/32), into the row-major layout the 8-wave kernels read with it
 * (kernels/gemm/inter_wave/a4w4/bench.py:110-115 builds such views).  No
 * counterpart in the reference.  G9_ERR_LAYOUT for null pointers or strides
 * below the row lengths; nothing is launched when rows or cols is 0.
 */
int g9_transpose_u8(const void* src, int64_t rows, int64_t cols, int64_t src_ld, void* dst, int64_t dst_ld,
                    void* stream);

/*
 * Name of the kernel a call with this (dtype, out_dtype, schedule, waves)
 * launches (for G9_SCHED_SPLITK: its segment kernel, followed by
 * g9_splitk_reduce_f16 or g9_splitk_reduce_bf16 by output type),
 * for profiler kernel filters (cf. KERNEL_NAME in
 * kernels/gemm/inter_wave/a8w8/matmul_kernel.py:52), or NULL.
 */
const char* g9_kernel_name(int dtype, int out_dtype, int schedule, int waves);

/* Human-readable text of a status code. */
const char* g9_status_string(int status);

/* Number of persistent workgroups the stream-K schedule launches on the current device. */
int g9_streamk_workgroups(void);

/*
 * K segments per tile the split-K schedule uses for `tiles` output tiles of
 * `stages` K stages on a device of `cus` CUs (1 = it runs as data-parallel).
 * Pure function of its arguments.  No counterpart in the reference.
 */
int g9_splitk_factor(int64_t tiles, int stages, int cus);

/* Library ABI version (major * 100 + minor). */
int g9_version(void);

#ifdef __cplusplus
}
#endif

#endif /* GFX950_GEMM_H */
