/*
 * awq_w4a16.h -- C ABI of the MI355X (gfx950) W4A16 AWQ GEMM library.
 *
 * The library replaces the GEMM behind kernels/awq_gemm.py::awq_gemm_forward
 * (kernels/awq_gemm.py:237-284) of Qwen2-7B-Triton_Engine.  Operand formats
 * are the reference's, unchanged:
 *
 *   x        fp16  [M, K]      row-major, contiguous
 *   qweight  int32 [K, N/8]    8 int4 codes per word; logical column n of a
 *                              word sits in nibble ORD[n % 8], ORD =
 *                              {0,4,1,5,2,6,3,7} (kernels/awq_gemm.py:5-6)
 *   qzeros   int32 [K/G, N/8]  zero codes, packed the same way
 *   scales   fp16  [K/G, N]
 *   out      fp16  [M, N]      out = x @ W, W[k,n] = fp16((q - z) * s),
 *                              accumulated in fp32, rounded once to fp16
 *
 * All pointers are device pointers.  `stream` is a hipStream_t (NULL = the
 * legacy default stream).  No entry point allocates device memory or
 * synchronises the host, and the only global state is looked up once per
 * device and then read (the device's compute-unit count; the address of the
 * allocation-free entry point's static scratch), so every call is reentrant
 * and can be captured into a HIP graph.  Every entry point returns AWQ_OK (0)
 * or a negative awq_w4a16_status.
 *
 * A GEMM call is one kernel launch, or two on the same stream when its plan
 * adds split-K partials in a second launch of a reduce kernel: tile
 * variants 7, 8 and 9 and stream variant 3 with split_k > 1.
 *
 * Numerics.  Every path computes in fp32 from the exact integer q - z.  The
 * tile paths and the per-weight skinny mode round each weight to fp16 as
 * the reference does (fp16((q - z) * s), one rounding, for every fp16
 * scale); the GEMV, stream and factored skinny paths multiply the fp32 sum
 * of x * (q - z) over a 128-row group by the scale instead (no per-weight
 * rounding: they stay finite where a reference weight would overflow).
 * The fixed-point split-K finish (GEMV variant 5, stream variant 1)
 * clamps each workgroup's partial sum to +-2^22 and turns a NaN partial
 * into +2^22, so a NaN or an infinity in x gives +-inf (never NaN) on those
 * paths -- except that a +inf and a -inf partial of different splits cancel,
 * so such an output can come out finite where the reference gives NaN.
 * The clamp can also change a finite result without a sign: partials of
 * opposite signs beyond 2^22 in magnitude (+5e6 and -4.99e6, say) are added
 * as +-2^22 and give 0 where the fp32 sum is about 1e4.  Partials that large
 * need |x| * |(q - z) * s| summed over one split's rows to exceed 4 million
 * (AWQ scales are below 1, q - z at most 15), far outside fp16 activations
 * of a working model; the other finishes have no such limit.  Partials are
 * added in 2^-24 steps.
 */
#ifndef AWQ_W4A16_H
#define AWQ_W4A16_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AWQ_W4A16_ABI_VERSION 2

typedef enum awq_w4a16_status {
    AWQ_OK = 0,
    AWQ_ERR_NULL_POINTER = -1,   /* a required pointer is NULL                        */
    AWQ_ERR_BAD_DIMS = -2,       /* M < 0, N <= 0, K <= 0, N % 8 != 0 or K % G != 0    */
    AWQ_ERR_GROUP_SIZE = -3,     /* group size other than 128                          */
    AWQ_ERR_MISALIGNED = -4,     /* x/out/scales not 16-byte, qweight/qzeros not 4-byte aligned */
    AWQ_ERR_WORKSPACE = -5,      /* workspace NULL or smaller than required            */
    AWQ_ERR_LAUNCH = -6,         /* the HIP runtime rejected a kernel launch           */
    AWQ_ERR_PATH = -7,           /* unknown kernel path, or path cannot serve this M   */
    AWQ_ERR_TOO_LARGE = -8,      /* M > 2^30, K > 2^22, N > 2^20 or operand > 2^31-1 B */
    AWQ_ERR_SCRATCH = -9,        /* awq_w4a16_gemm_noalloc: workspace > the static scratch */
    AWQ_ERR_CAPTURE = -10        /* awq_w4a16_gemm_noalloc: first split-K call on a device under capture */
} awq_w4a16_status;

/* Kernel paths.  AUTO lets the shape dispatcher choose (the reference's own
 * choice is by M alone, kernels/awq_gemm.py:251); the others force one
 * kernel family, for tests and measurements. */
typedef enum awq_w4a16_path {
    AWQ_PATH_AUTO = 0,
    AWQ_PATH_SKINNY = 1,         /* decode: MFMA skinny-M streaming kernel (M <= 64)         */
    AWQ_PATH_TILE = 2,           /* prefill: LDS-tiled MFMA GEMM                            */
    AWQ_PATH_GEMV = 3,           /* decode: column-strip GEMV (quads, pairs, singles), MFMA
                                    or dot2 sums; M <= 2 when forced, to 16 under AUTO     */
    AWQ_PATH_STREAM = 5          /* decode: streaming 16x16x32 MFMA kernels (M <= 16)       */
} awq_w4a16_path;

/* What the dispatcher will launch for a shape (host-side description). */
typedef struct awq_w4a16_plan {
    int32_t path;                /* AWQ_PATH_SKINNY, _TILE, _GEMV or _STREAM                */
    int32_t variant;             /* kernel variant inside the path                          */
    int32_t tile_m;              /* rows of x per work unit (skinny: 16, 32 or 64; gemv:
                                    the rows of x its instance carries)                    */
    int32_t tile_n;              /* output columns per work unit                            */
    int32_t rows_per_wave;       /* skinny: K rows per wavefront (32, 64 or 128*q)          */
    int32_t k_waves;             /* skinny: wavefronts per workgroup along K (1, 2, 4)      */
    int32_t split_k;             /* workgroups along K; > 1 uses the fp32 workspace         */
    int32_t block_threads;       /* threads per workgroup                                   */
    int32_t factored_scale;      /* skinny: 1 = scale applied per group sum, 0 = per weight */
    int32_t depth;               /* gemv, stream: chunk buffers per wave (gemv variant 2:
                                    128-row groups in flight); else 0                      */
    int64_t grid;                /* workgroups in the one launch                            */
    uint64_t workspace_bytes;    /* split_k > 1: counter block + 64-bit fixed-point slots
                                    or counters + slot region + fp32 partials; else 0    */
    uint64_t lds_bytes;          /* dynamic LDS per workgroup                               */
} awq_w4a16_plan;

/* ABI version of the loaded library (AWQ_W4A16_ABI_VERSION).  No reference
 * counterpart; lets a binding refuse a mismatched library. */
int awq_w4a16_abi_version(void);

/* Static text for a status code.  No reference counterpart (the reference
 * raises no errors for bad operands, kernels/awq_gemm.py:237-284). */
const char* awq_w4a16_error_string(int status);

/* Host-only: fill *plan with what awq_w4a16_gemm_ex would launch for this
 * shape and path, after validating the dimensions.  Launches nothing; grids
 * and split counts are sized for the compute units of the current device
 * (read once per device; 256, an MI355X, where no device is visible), so a
 * plan made for one device should be launched on a device of the same kind.
 * Replaces the M-based dispatch of kernels/awq_gemm.py:251 (M <= 4 ->
 * dequant + cuBLAS, else the autotuned Triton GEMM of :152-164). */
int awq_w4a16_plan_for(int64_t M, int64_t N, int64_t K, int32_t group_size,
                       int32_t path, awq_w4a16_plan* plan);

/* Host-only: a skinny-path plan with explicit tuning values (rows_per_wave:
 * 32, 64 or a multiple of 128 not above K; k_waves: 1, 2 or 4; variant: 1
 * pipelined or 2 plain main loop; factored_scale: 0 or 1), with the derived
 * fields (split_k, grid, workspace and LDS bytes) filled in.  For sweeps;
 * AWQ_ERR_PATH if the values cannot serve the shape. */
int awq_w4a16_plan_skinny(int64_t M, int64_t N, int64_t K, int32_t group_size,
                          int32_t rows_per_wave, int32_t k_waves, int32_t variant,
                          int32_t factored_scale, awq_w4a16_plan* plan);

/* Host-only: a tile-path plan.  Variant 6: 128x256x64 tiles (four
 * wavefronts, two workgroups per CU), each wavefront 128 x rows x 64
 * columns, weights dequantised straight into MFMA operand registers, x, raw
 * weights and zeros/scales brought by direct global->LDS loads two k-steps
 * ahead into a 3-stage ring, the last-arriving split adding the split-K
 * partials; variants 7, 8, 9: 128-, 64- and 32-row tiles of the same kernel
 * (two, three, four workgroups per CU) whose split-K partials are summed by
 * a second, whole-device launch; variants 13, 14: hybrids of variants 6 and
 * 8 for grids that do not divide the CUs -- `full` whole tiles on every CU
 * (fewer than a CU holds: one for 13, one or two for 14) and the L leftover
 * tiles split split_k >= 2 ways along K, at most one piece per CU (grid =
 * full x CUs + L x split_k), the pieces' partials compact ([split_k, L,
 * rows, 256] fp32) and added by each leftover tile's last-arriving piece;
 * other shapes get AWQ_ERR_PATH; variant 15: variant 7 with eight
 * wavefronts on 128 x 512 tiles (one workgroup per CU, x rows loaded once
 * per 512 columns), bit-identical to variant 7 at the same split_k (plan
 * tile_n 512, block_threads 512).  Every variant takes split_k >= 1
 * workgroups along K in whole 128-row groups; the plan's rows_per_wave holds
 * the K rows per split.  Other variant numbers (1 .. 5 and the retired
 * 10 .. 12 included): AWQ_ERR_PATH. */
int awq_w4a16_plan_tile(int64_t M, int64_t N, int64_t K, int32_t group_size,
                        int32_t variant, int32_t split_k, awq_w4a16_plan* plan);

/* Host-only: a GEMV-path plan with explicit tuning values.
 * variant 5 (N % 32 == 0, column sums on v_mfma_f32_16x16x32_f16): tile_n
 * is the strip width -- 512 (column quads, M <= 2, depth 2 .. 4), 256
 * (column pairs, M <= 4) or 128 (column singles, M <= 8; pairs and singles
 * depth 2 .. 3);
 * rows_per_wave 0; depth = chunk buffers per wavefront (depth - 1 chunks of
 * loads in flight while one is computed); k_waves 1 .. 8 wavefronts, which
 * take every k_waves-th 32-row chunk of the workgroup's share of K; split_k
 * 1 .. min(K/32, 255) workgroups share each strip's K evenly; split-K
 * partials meet in 64-bit fixed-point workspace slots.
 * variant 6: column singles (tile_n 128) with 16 rows of x, 9 <= M <= 16,
 * depth 2, k_waves and split_k as variant 5; split-K partials are fp32
 * ([split_k, M, N] in the workspace) added by a second launch.
 * variant 2 (K-streaming, one 128-row group per step): tile_n 512;
 * rows_per_wave 16 or 32, k_waves = 128 / rows_per_wave, split_k in
 * 1 .. K/128 with every split a whole number of groups, depth = chunks in
 * flight per wave (2 .. 4 for 16 rows per wave, 2 .. 3 for 32).
 * Other variants: AWQ_ERR_PATH. */
int awq_w4a16_plan_gemv(int64_t M, int64_t N, int64_t K, int32_t group_size, int32_t variant,
                        int32_t tile_n, int32_t rows_per_wave, int32_t k_waves, int32_t split_k,
                        int32_t depth, awq_w4a16_plan* plan);

/* Host-only: a stream-path plan (M <= 16, N % 32 == 0): each 64-packed-
 * column strip's K/128 groups are divided evenly among split_k workgroups
 * (1 .. K/128) whose wavefronts take every k_waves-th group;
 * v_mfma_f32_16x16x32_f16 sums x * (1024 + q) and x per group, zero and
 * scale fold in once per group in fp32.  rows_per_wave 16: row layout
 * (M <= 8), every load covers whole 256-byte row segments and the two
 * column halves share one MFMA through the rows of A; k_waves wavefronts
 * share every group: k_waves 1, 2, 4 or 8 with depth 2 chunk buffers per
 * wavefront or 4 or 8 with depth 1.  rows_per_wave 32: half-strip layout (M <= 16),
 * the two wavefronts of a pair read the two halves of each row segment;
 * k_waves pairs, 1 .. 4 with depth 2, 1 .. 2 with depth 4 or 6.  Split-K
 * finish: variant 1, 64-bit fixed-point workspace slots (one atomic per
 * output element per workgroup; split_k <= 255); variant 2, fp32 partials
 * added by the last-arriving workgroup of each strip; variant 3, fp32
 * partials added by a second kernel launch on the same stream.  No
 * reference counterpart beyond the decode dispatch it serves
 * (kernels/awq_gemm.py:251-282). */
int awq_w4a16_plan_stream(int64_t M, int64_t N, int64_t K, int32_t group_size, int32_t rows_per_wave,
                          int32_t variant, int32_t k_waves, int32_t split_k, int32_t depth,
                          awq_w4a16_plan* plan);
/* Bytes of the fixed-point slot region of a workspace (see below). */
#define AWQ_W4A16_SLOT_BYTES ((size_t)2 << 20)

/* Host-only: bytes of workspace awq_w4a16_gemm needs for this shape
 * (0 if none).  Replaces the module-global _dequant_buffer of
 * kernels/awq_gemm.py:234,255-262, which holds K*N fp16 values.  The
 * workspace of a split-K launch is laid out as
 *   [uint32 arrival counters: awq_w4a16_counter_bytes()]
 *   [64-bit fixed-point slots, one per output element [M, N]: at most
 *    AWQ_W4A16_SLOT_BYTES (GEMV variant 5 and stream variant 1)]
 *   [fp32 partial sums (every other split-K plan): [split_k, M, N]; for
 *    tile variants 7, 8, 9 and 15 units of 16 rows x 256 columns in the MFMA
 *    accumulators' lane order, [split_k, ceil(M/16), ceil(N/256), 16 KB];
 *    for the hybrid tile variants 13 and 14 only the leftover tiles',
 *    [split_k, leftover tiles, tile rows, 256]]
 * and its size is the end of the last region the plan uses.  The counters
 * and slots must be zero-filled before the first call and every call leaves
 * them zero; the partials region is never cleared (each call writes every
 * partial it reads).  So one workspace zero-filled once serves any number of
 * calls of any path, as long as calls that share it do not run
 * concurrently.  Returns 0 for invalid dimensions as well;
 * awq_w4a16_plan_for reports the reason. */
size_t awq_w4a16_counter_bytes(void);
size_t awq_w4a16_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t group_size);
size_t awq_w4a16_workspace_bytes_ex(int64_t M, int64_t N, int64_t K, int32_t group_size,
                                    int32_t path);

/* Host-only: the checks awq_w4a16_gemm_ex performs before launching
 * (pointers, dimensions, alignment, workspace size), without launching. */
int awq_w4a16_validate(const void* x, const void* qweight, const void* qzeros,
                       const void* scales, const void* out, int64_t M, int64_t N,
                       int64_t K, int32_t group_size, const void* workspace,
                       size_t workspace_bytes, int32_t path);

/* out[M,N] = x[M,K] @ dequant(qweight, qzeros, scales).
 * Replaces awq_gemm_forward (kernels/awq_gemm.py:237-284) for a flattened
 * x (:244-246); the caller allocates `out` (the reference allocates it,
 * :249) and, when awq_w4a16_workspace_bytes() > 0, `workspace`.
 * M == 0 is a valid no-op. */
int awq_w4a16_gemm(const void* x, const int32_t* qweight, const int32_t* qzeros,
                   const void* scales, void* out, int64_t M, int64_t N, int64_t K,
                   int32_t group_size, void* workspace, size_t workspace_bytes,
                   void* stream);

/* As awq_w4a16_gemm, with the kernel path forced (AWQ_PATH_*).  The
 * workspace must be at least awq_w4a16_workspace_bytes_ex(..., path). */
int awq_w4a16_gemm_ex(const void* x, const int32_t* qweight, const int32_t* qzeros,
                      const void* scales, void* out, int64_t M, int64_t N, int64_t K,
                      int32_t group_size, void* workspace, size_t workspace_bytes,
                      int32_t path, void* stream);

/* As awq_w4a16_gemm_ex, launching a caller-supplied plan: one from
 * awq_w4a16_plan_for, or one filled by awq_w4a16_plan_skinny with other
 * tuning values.  The plan is checked against the
 * shape first (AWQ_ERR_PATH if inconsistent).  Replaces the per-(M,N,K)
 * autotuning of kernels/awq_gemm.py:152-164 with an explicit, stateless
 * choice the caller can sweep. */
int awq_w4a16_gemm_planned(const void* x, const int32_t* qweight, const int32_t* qzeros,
                           const void* scales, void* out, int64_t M, int64_t N, int64_t K,
                           int32_t group_size, void* workspace, size_t workspace_bytes,
                           const awq_w4a16_plan* plan, void* stream);

/* Bytes of the per-device static scratch of awq_w4a16_gemm_noalloc. */
#define AWQ_NOALLOC_SCRATCH_BYTES (32u << 20)

/* As awq_w4a16_gemm, allocating nothing and taking no workspace argument.
 * No reference counterpart: it is for callers that cannot allocate device
 * memory -- code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc.  The split-K workspace is a static device array of
 * AWQ_NOALLOC_SCRATCH_BYTES (32 MiB) that the library holds on every GPU it
 * runs on until the process ends.  The first call on a device that needs a
 * split-K workspace looks up the device's address of the array (the device
 * `stream` belongs to), clears its counter and slot regions with one fill
 * kernel on `stream` and waits for it; that first call must not be made
 * under graph capture (AWQ_ERR_CAPTURE: make one eager call on each device
 * before capturing), later calls may be captured.  The plan is the AUTO
 * plan, except that a tile plan whose workspace would exceed the scratch
 * takes the largest split-K count that fits (so results can differ from
 * awq_w4a16_gemm in the last bits there); a decode plan that does not fit
 * (M * N beyond about a million outputs) returns AWQ_ERR_SCRATCH.  Every
 * call on a GPU shares that GPU's scratch, which each call leaves zero:
 * calls that overlap on one GPU (other streams, other threads) race. */
int awq_w4a16_gemm_noalloc(const void* x, const int32_t* qweight, const int32_t* qzeros,
                           const void* scales, void* out, int64_t M, int64_t N, int64_t K,
                           int32_t group_size, void* stream);

/* w[K,N] fp16 = fp16((q - z) * s), the dense dequantised weight, bit-exact.
 * Replaces _dequant_to_fp16 / _dequant_awq_kernel (kernels/awq_gemm.py:14-87);
 * it runs the same unpack/dequant device code as the GEMM kernels. */
int awq_w4a16_dequant(const int32_t* qweight, const int32_t* qzeros, const void* scales,
                      void* w_out, int64_t N, int64_t K, int32_t group_size, void* stream);

/* The GEMM with the reference's elementwise follow-ups fused into its final
 * store: out = fp16(x @ W), then + bias[n] when bias is non-NULL, then
 * + residual[m, n] when residual is non-NULL, each add done in fp32 and
 * rounded to fp16 -- bit-identical to awq_w4a16_gemm followed by the
 * reference's `out + bias` (QKV bias, model/qwen2.py:45-46,108-109) and
 * `residual + out` (after o_proj / down_proj, :219-227) on torch fp16
 * tensors, without their two extra passes over [M, N].  bias is fp16 [N],
 * residual fp16 [M, N] (2-byte aligned; residual may alias out).  plan NULL
 * = the AUTO plan (as awq_w4a16_gemm), else a plan from awq_w4a16_plan_*
 * checked against the shape (as awq_w4a16_gemm_planned). */
int awq_w4a16_gemm_epilogue(const void* x, const int32_t* qweight, const int32_t* qzeros,
                            const void* scales, const void* bias, const void* residual, void* out,
                            int64_t M, int64_t N, int64_t K, int32_t group_size, void* workspace,
                            size_t workspace_bytes, const awq_w4a16_plan* plan, void* stream);

/* out[m, i] = fp16(silu(g) * u), g = gate_up[m, i], u = gate_up[m, I + i], in
 * fp32 with one rounding: the reference's silu_mul (kernels/silu_mul.py:17-39)
 * over the fused gate||up projection read in place, replacing its two
 * .contiguous() copies and the silu_mul pass (model/qwen2.py:187-194) by one
 * pass.  gate_up fp16 [M, 2I], out fp16 [M, I], both 16-byte aligned,
 * I % 8 == 0. */
int awq_silu_mul(const void* gate_up, void* out, int64_t M, int64_t I, void* stream);

/* out[M,N] = x[M,K] @ weight[N,K]^T in fp16 with fp32 accumulation (one
 * v_mfma_f32_16x16x32_f16 per 16 weight rows x 32 k): the
 * fp16 output projection (lm_head) of model/qwen2.py:253,280
 * (nn.Linear(hidden_size, vocab_size, bias=False), applied at :280), at
 * decode sizes.  weight is nn.Linear's row-major [out_features, in_features]
 * fp16.  M in 0 .. 8 (AWQ_ERR_PATH above: greedy decoding needs the last
 * position only); K % 8 == 0 and K <= 4096 (AWQ_ERR_BAD_DIMS /
 * AWQ_ERR_TOO_LARGE); x and weight 16-byte aligned.
 * No workspace; M == 0 is a valid no-op. */
int awq_fp16_linear(const void* x, const void* weight, void* out, int64_t M, int64_t N, int64_t K,
                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AWQ_W4A16_H */
