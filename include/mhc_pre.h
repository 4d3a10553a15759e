/*
 * MhcPre for AMD Instinct MI355X (gfx950): C ABI.
 *
 * MhcPre is the pre-mixing step of a multi-stream (hyper-connection) residual
 * block.  For every token row r of x [T, n, D] (T = B*S, K = n*D,
 * M = n*n + 2n):
 *
 *   invRms  = 1 / sqrt(sum_k x[r,k]^2 / K + normEps)
 *   mix[j]  = sum_k (x[r,k] * gamma[k]) * phi_mem[j*K + k]          (j < M)
 *   hPre[i] = sigmoid(mix[i]     * (invRms*alpha[0]) + bias[i])     + hcEps
 *   hPost[i]= 2 * sigmoid(mix[n+i] * (invRms*alpha[1]) + bias[n+i])
 *   hRes[i*n+j] = mix[2n+i*n+j] * (invRms*alpha[2]) + bias[2n+i*n+j]
 *   hIn[r,d]= RNE_dtype(sum_s hPre[s] * x[r,s,d])
 *
 * The API mirrors the reference operator's generated two-phase aclnn API
 * (aclnnMhcPreGetWorkspaceSize / aclnnMhcPre, as called at
 * cloud_runner/runner.cpp:443-445,459): phase 1 validates the tensors, sizes
 * the device workspace and returns an executor bound to the tensors' device
 * addresses; phase 2 launches on a HIP stream.  The caller owns every device
 * buffer, including the workspace, whose contents need not be preserved
 * between launches.  An executor's plan is immutable after creation (it only
 * records the id of its latest launch, for mhcPreQueryDeviceStatus): it may
 * be launched any number of times (the reference probe relaunches one
 * executor, cloud_runner/probe_e1e2.cpp:312-326) and from several host threads
 * on different streams, provided the launches do not share a workspace
 * concurrently.  No function aborts; every failure is a status code.
 */
#ifndef MHC_PRE_H
#define MHC_PRE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Exported symbols (the library is built with hidden default visibility). */
#ifndef MHC_API
#define MHC_API __attribute__((visibility("default")))
#endif

/* Same declaration as HIP's runtime header, so callers need no HIP include. */
typedef struct ihipStream_t *hipStream_t;

/* Element types.  The values are those of the reference stack's aclDataType
 * (ACL_FLOAT = 0, ACL_FLOAT16 = 1, ACL_BF16 = 27) so a binding can pass them
 * through unchanged. */
#define MHC_DTYPE_FLOAT 0
#define MHC_DTYPE_FLOAT16 1
#define MHC_DTYPE_BF16 27

#define MHC_MAX_DIMS 8

/* A dense row-major tensor over caller-owned device memory (aclTensor's role,
 * cloud_runner/runner.cpp:217-218).  `data` may be NULL only for an absent
 * optional tensor or one with zero elements. */
typedef struct mhcTensor {
    void *data;
    int32_t dtype;
    int32_t ndim;
    int64_t dims[MHC_MAX_DIMS];
} mhcTensor;

typedef struct mhcPreExecutor mhcPreExecutor;

/* Status codes (0 = success, like ACL_SUCCESS). */
#define MHC_STATUS_SUCCESS 0
#define MHC_STATUS_NULL_ARGUMENT 1        /* a required pointer is NULL */
#define MHC_STATUS_INVALID_SHAPE 2        /* rank / dims / element counts inconsistent */
#define MHC_STATUS_UNSUPPORTED_SHAPE 3    /* n not in {4,6,8}, D % 16, n*D % 8, M > 80,
                                             B*S >= 2^28 rows, D > 2^24 */
#define MHC_STATUS_INVALID_DTYPE 4        /* x not fp16/bf16, fp32 tensors not fp32, hIn != x */
#define MHC_STATUS_WORKSPACE_TOO_SMALL 5  /* workspace NULL or smaller than phase 1 asked */
#define MHC_STATUS_HIP_ERROR 6            /* a HIP runtime call failed */
#define MHC_STATUS_DEVICE_MISMATCH 7      /* phase 2 called with another device current than
                                             the one holding x at phase 1 */
#define MHC_STATUS_DEVICE_TIMEOUT 8       /* a kernel's bounded inter-workgroup wait expired */
#define MHC_STATUS_MISALIGNED 9           /* x, hIn, phi, gamma not 16-byte aligned; others not 4 */
#define MHC_STATUS_SCRATCH_TOO_SMALL 10   /* mhcPreNoAlloc: the executor needs a workspace larger
                                             than the built-in scratch (64 MiB) */

/*
 * Phase 1.  Replaces aclnnMhcPreGetWorkspaceSize (argument list and meaning
 * as cloud_runner/runner.cpp:443-445; validation rules of the reference
 * TilingFunc, code/op_host/mhc_pre.cpp:57-79,126-130; output shapes of its
 * InferShape / InferDataType, code/op_host/mhc_pre.cpp:217-257).
 *
 *   x      fp16 | bf16  [B, S, n, D]  (a 3-D [T, n, D] is accepted as an extension)
 *   phi    fp32         n*D*M elements, read as memory [M][K] (phi_mem[j*K + k])
 *   alpha  fp32         3 elements {alphaPre, alphaPost, alphaRes}
 *   bias   fp32         M elements: [0,n) pre, [n,2n) post, [2n, 2n+n*n) res
 *   gamma  fp32         n*D elements, or NULL / zero elements => gamma off
 *                       (code/op_host/mhc_pre.cpp:90)
 *   normEps, hcEps      the op attributes (reference defaults 1e-6,
 *                       code/op_host/mhc_pre.cpp:297-298)
 *   hIn    dtype of x   [B, S, D]
 *   hPost  fp32         [B, S, n]
 *   hRes   fp32         [B, S, n, n]
 * On success *workspaceSize holds the bytes the caller must allocate and
 * *executor a new executor (free it with mhcPreExecutorDestroy).  The size is
 * that of the launch path the plan takes.  On the strip path (n = 4, D a
 * multiple of 32 from 192 up to 16384, all but small batches) it holds per-team
 * exchange rings only and does not grow with T (7.2 MB at n = 4, D = 7168);
 * the team count is that of the device holding x (of MI355X when the runtime
 * cannot tell).  The two-pass paths hold partial sums that grow with T.
 */
MHC_API int mhcPreGetWorkspaceSize(const mhcTensor *x, const mhcTensor *phi, const mhcTensor *alpha,
                           const mhcTensor *bias, const mhcTensor *gamma, float normEps,
                           float hcEps, const mhcTensor *hIn, const mhcTensor *hPost,
                           const mhcTensor *hRes, uint64_t *workspaceSize,
                           mhcPreExecutor **executor);

/*
 * Phase 1 with one extra optional output, hPre fp32 [B, S, n] (NULL => not
 * written).  Extension: the reference keeps hPre on chip only
 * (code/op_kernel/mhc_pre.cpp:742-750); everything else is as
 * mhcPreGetWorkspaceSize.
 */
MHC_API int mhcPreGetWorkspaceSizeWithHPre(const mhcTensor *x, const mhcTensor *phi,
                                   const mhcTensor *alpha, const mhcTensor *bias,
                                   const mhcTensor *gamma, float normEps, float hcEps,
                                   const mhcTensor *hIn, const mhcTensor *hPost,
                                   const mhcTensor *hRes, const mhcTensor *hPre,
                                   uint64_t *workspaceSize, mhcPreExecutor **executor);

/*
 * Phase 2.  Replaces aclnnMhcPre (cloud_runner/runner.cpp:459,472): enqueues
 * the operator on `stream` (NULL = the null stream) and returns without
 * waiting.  The workspace must hold at least the bytes phase 1 returned.  The
 * device holding the tensors must be the current device
 * (MHC_STATUS_DEVICE_MISMATCH otherwise), as aclnn launches run on the
 * context's device.  A strip executor on a device that cannot co-schedule the
 * teams phase 1 planned for (which MI355X always can) runs a fallback path only
 * if the workspace holds that path's layout, and returns
 * MHC_STATUS_UNSUPPORTED_SHAPE otherwise.
 *
 * The strip and fused kernels' workgroups wait on each other (bounded), so
 * their grids are sized to what the device holds at once.  By default it is a
 * plain launch: every workgroup is resident unless another kernel occupies the
 * device at the same time, in which case a wait can expire: the launch still
 * ends (no hang), mhcPre has already returned MHC_STATUS_SUCCESS, the rows
 * whose wait expired hold NaN in hIn / hPre / hPost / hRes (never a plausible
 * value), and mhcPreQueryDeviceStatus reports MHC_STATUS_DEVICE_TIMEOUT.  With
 * the environment variable MHCPRE_LAUNCH=cooperative at phase 1 the executor
 * uses a cooperative launch, which guarantees co-residency next to concurrent
 * work but dispatches more slowly (about 20 us per launch on MI355X).
 *
 * A launch may be captured into a HIP graph and replayed: the exchange epoch
 * that tells the current launch's data from stale workspace contents is kept
 * in the workspace itself and advanced by every launch, replays included.
 */
MHC_API int mhcPre(void *workspace, uint64_t workspaceSize, mhcPreExecutor *executor,
           hipStream_t stream);

/*
 * Prepared weights.  Extension; the reference rebuilds its GEMM operand from
 * phi and gamma on every launch (the gamma product in PreprocessRows and the
 * phi read of ProjectWithCube, code/op_kernel/mhc_pre.cpp:466-468,535, with
 * the per-call tiling of code/op_host/mhc_pre.cpp:159-177).  For weights that
 * stay fixed over many launches, mhcPrePrepareWeights computes
 * B = gamma (.) phi once, split into bf16 hi + lo MFMA fragments, into a
 * caller-owned device buffer; executors created from it
 * (mhcPreGetWorkspaceSizePrepared) copy or read those fragments instead of
 * building them from phi and gamma on every launch.  Results are bit-identical
 * to executors built from phi and gamma.
 *
 * `n` is the stream count (4, 6 or 8; M = n*n + 2n); phi is fp32 with K*M
 * elements (memory [M][K], as for phase 1), gamma fp32 with K elements or
 * NULL / zero elements for none.  The buffer must hold
 * mhcPrePrepareWeightsSize bytes (K * 2M * 2), be 256-byte aligned and live on
 * the current device.  The preparation is enqueued on `stream`; launches on
 * other streams must be ordered after it by the caller.
 *
 * `version` is the caller's key for the weights the buffer holds (for example
 * an update counter); mhcPreWeightsVersion returns it.  Preparing again into
 * the same buffer (same shapes) updates, from their next launch on, every
 * executor created from that buffer; the buffer must outlive them, the
 * weights object need not.
 */
typedef struct mhcPreWeights mhcPreWeights;

MHC_API int mhcPrePrepareWeightsSize(const mhcTensor *phi, const mhcTensor *gamma, int32_t n,
                                     uint64_t *bytes);

MHC_API int mhcPrePrepareWeights(const mhcTensor *phi, const mhcTensor *gamma, int32_t n,
                                 void *buffer, uint64_t bytes, uint64_t version,
                                 hipStream_t stream, mhcPreWeights **weights);

MHC_API int mhcPreWeightsVersion(const mhcPreWeights *weights, uint64_t *version);

MHC_API int mhcPreWeightsDestroy(mhcPreWeights *weights);

/*
 * Phase 1 from prepared weights: as mhcPreGetWorkspaceSizeWithHPre with phi
 * and gamma replaced by `weights` (x's n must be the prepared n and its n*D
 * the prepared K; MHC_STATUS_INVALID_SHAPE otherwise).  hPre may be NULL.
 * The executor reads the weights' buffer at every launch.
 */
MHC_API int mhcPreGetWorkspaceSizePrepared(const mhcTensor *x, const mhcPreWeights *weights,
                                           const mhcTensor *alpha, const mhcTensor *bias,
                                           float normEps, float hcEps, const mhcTensor *hIn,
                                           const mhcTensor *hPost, const mhcTensor *hRes,
                                           const mhcTensor *hPre, uint64_t *workspaceSize,
                                           mhcPreExecutor **executor);

/*
 * Phase 2 without a caller workspace.  No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  As mhcPre, but the
 * workspace is a fixed 64 MiB array built into the library, one per device,
 * held until the process ends; the call allocates nothing.  An executor whose
 * phase-1 workspace size exceeds 64 MiB is rejected with
 * MHC_STATUS_SCRATCH_TOO_SMALL (every workload up to n=4, D=7168, T=8192 and
 * n=8, D=8192, T=5472 fits).  All calls on one device share that device's
 * array: calls that overlap on a device (other streams, other host threads)
 * race and must be ordered by the caller.  An expired wait between
 * workgroups shows as NaN in the affected outputs (the status word lives in
 * the built-in array, which mhcPreQueryDeviceStatus does not read).
 */
MHC_API int mhcPreNoAlloc(mhcPreExecutor *executor, hipStream_t stream);

/* Releases an executor (the generated aclnn API frees executors itself). */
MHC_API int mhcPreExecutorDestroy(mhcPreExecutor *executor);

/*
 * Device-side status of this executor's latest launch on `workspace`:
 * MHC_STATUS_SUCCESS, or MHC_STATUS_DEVICE_TIMEOUT if one of its bounded
 * waits between workgroups expired (the outputs of such a launch are not
 * valid).  Synchronizes `stream` first.  workspace NULL with workspaceSize 0
 * reads the current device's built-in workspace, that of mhcPreNoAlloc
 * launches.  No reference counterpart (the reference detects a hang only by
 * the caller's own wait, cloud_runner/probe_e1e2.cpp:295).
 */
MHC_API int mhcPreQueryDeviceStatus(void *workspace, uint64_t workspaceSize,
                            const mhcPreExecutor *executor, hipStream_t stream);

/*
 * A sticky device status word for the executor's launches, read without an
 * extra synchronize.  No reference counterpart: for callers that launch
 * without waiting (graph replays, serving loops) and check for errors at
 * their own next synchronization.  From the executor's next launch on, a
 * strip or fused launch whose bounded wait between workgroups expired (its
 * rows then hold NaN) stores MHC_STATUS_DEVICE_TIMEOUT into *deviceWord, a
 * 4-byte-aligned word of device memory on the executor's device; nothing
 * else ever writes it, so the caller zeroes it, reads it after any later
 * synchronization of its own, and zeroes it again.  One word may serve many
 * executors.  deviceWord NULL turns it off.  Set it before launching, not
 * concurrently with launches of the same executor.  Such an expiry needs
 * another kernel to hold CUs the launch needs (an RCCL kernel on a
 * communication stream, say) and is turned into a guarantee by
 * MHCPRE_LAUNCH=cooperative.
 */
MHC_API int mhcPreExecutorSetStatusWord(mhcPreExecutor *executor, uint32_t *deviceWord);

/* Human-readable name of a status code (static storage). */
MHC_API const char *mhcPreStatusString(int status);

/* Which kernel path an executor launches (diagnostics and benchmarks):
 * writes a static NUL-terminated name to *name. */
MHC_API int mhcPreExecutorPath(const mhcPreExecutor *executor, const char **name);

/*
 * Measurement aid, no counterpart in the reference: enqueues one launch of a
 * stream kernel that reads `readBytes` from `src` and writes `writeBytes` to
 * `dst` with no arithmetic, in the access pattern the device serves best
 * (whole 1 KB wavefront loads and stores, 4 KB read blocks, grid-strided).
 * Timing it gives a measured bandwidth ceiling for a byte mix, e.g. the
 * operator's x read and hIn write, to set beside the operator's own rate.
 * readBytes must be a multiple of 4096 and writeBytes of 1024 (otherwise
 * MHC_STATUS_INVALID_SHAPE); src and dst 16-byte aligned.  `workgroups`
 * workgroups of 512 threads, 0 for one per compute unit.  The written data is
 * a function of the read data and has no other meaning.
 */
MHC_API int mhcPreStreamProbe(const void *src, uint64_t readBytes, void *dst, uint64_t writeBytes,
                              int32_t workgroups, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MHC_PRE_H */
