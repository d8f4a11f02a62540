/* C ABI of the MI355X (gfx950) Gated Delta Network kernels.
 *
 * Shape contract (fixed by the reference definitions gdn_decode_qk4_v8_d128_k_last
 * and gdn_prefill_qk4_v8_d128_k_last): 4 q/k heads, 8 v heads (v-head h reads
 * q/k head h/2), head dim K = V = 128, k-last fp32 state [N, 8, V=128, K=128].
 * All tensors are dense row-major device buffers.  bf16 buffers are passed as
 * untyped pointers to 16-bit words.  Every entry point is asynchronous on
 * `stream` (a hipStream_t; NULL = the default stream), performs no host
 * synchronisation and allocates nothing.  Return value: GDN_OK, a negative
 * GDN_ERR_* code for rejected arguments (nothing launched), or a positive
 * hipError_t from the launch.
 */
#ifndef GDN_MI355X_H
#define GDN_MI355X_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GDN_ABI_VERSION 2

enum {
  GDN_OK = 0,
  GDN_ERR_INVALID_ARGUMENT = -1,   /* null pointer, negative size, bad option */
  GDN_ERR_WORKSPACE_TOO_SMALL = -2,
  GDN_ERR_UNALIGNED = -3,          /* a buffer misses its required alignment */
  GDN_ERR_ALIASING = -4,           /* state and new_state are the same buffer */
  GDN_ERR_TOO_LARGE = -5           /* batch needs more than the no-allocation scratch */
};

/* Size of the device scratch array behind gdn_prefill_fwd_noalloc (per GPU). */
#define GDN_PREFILL_NOALLOC_SCRATCH_BYTES (128u << 20)

/* ABI version of the loaded library (GDN_ABI_VERSION it was built with). */
int gdn_abi_version(void);

/* Static text for a status code returned by the entry points. */
const char* gdn_status_string(int status);

/* Decode: one token for each of `batch` sequences.
 *
 * Replaces launch_gdn(q, k, v, state, A_log, a, dt_bias, b, scale, out, new_state)
 * of gdn_decode_qk4_v8_d128_k_last/solution/cuda/kernel.cu:982-1064 (argument
 * order kept); results follow solution/reference_torch_impl.py:11-72.
 *   q, k      [batch, 1, 4, 128] bf16   (8-byte aligned)
 *   v         [batch, 1, 8, 128] bf16   (2-byte aligned, as are a, b, out)
 *   state     [batch, 8, 128, 128] fp32 (16-byte aligned; read only)
 *   A_log     [8] fp32,  dt_bias [8] fp32 (4-byte aligned)
 *   a, b      [batch, 1, 8] bf16
 *   scale     output scale; 0 selects 1/sqrt(128)
 *   out       [batch, 8, 128] bf16 (written)
 *   new_state [batch, 8, 128, 128] fp32 (16-byte aligned; written; must not be `state`)
 *   rows_per_wave  state rows per wave64 work-group: 16 or 32, 0 = automatic
 */
int gdn_decode_fwd(const void* q, const void* k, const void* v, const float* state,
                   const float* A_log, const void* a, const float* dt_bias, const void* b,
                   float scale, void* out, float* new_state, int batch, int rows_per_wave,
                   void* stream);

/* Default workspace size in bytes for gdn_prefill_fwd with `num_seqs` sequences
 * and `total_tokens` tokens (the caller allocates it; its contents on entry are
 * irrelevant).  The reference allocates the same kind of scratch per call with
 * torch.empty (gdn_prefill_qk4_v8_d128_k_last/solution/triton/kernel.py:132-218).
 * About 2.9 KiB per token plus up to 48 MiB of segment slots (1 MiB each); a
 * larger workspace gives the planner more slots, a smaller one (down to
 * gdn_prefill_workspace_min_bytes) fewer.  Results do not depend on it. */
size_t gdn_prefill_workspace_bytes(int num_seqs, long long total_tokens);

/* Smallest workspace gdn_prefill_fwd accepts: no segment slots, so no sequence
 * is cut into segments that run concurrently (long sequences run their chunks
 * one after the other).  No reference counterpart: it states the floor of the
 * workspace contract above. */
size_t gdn_prefill_workspace_min_bytes(int num_seqs, long long total_tokens);

/* Prefill: chunked recurrence over a cu_seqlens ragged batch.
 *
 * Replaces launch_gdn(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale,
 * output, new_state) of gdn_prefill_qk4_v8_d128_k_last/solution/triton/kernel.py:56-262
 * (argument order kept); results follow solution/reference_torch_impl.py:16-92,
 * including new_state = 0 for an empty sequence.
 *   q, k        [total_tokens, 4, 128] bf16 (16-byte aligned)
 *   v           [total_tokens, 8, 128] bf16 (16-byte aligned)
 *   state       [num_seqs, 8, 128, 128] fp32 or NULL for zeros (16-byte aligned)
 *   A_log, dt_bias [8] fp32 (4-byte aligned);  a, b [total_tokens, 8] bf16 (2-byte aligned)
 *   cu_seqlens  [num_seqs + 1] int32 (cu_seqlens_is_int64 == 0) or int64, naturally aligned;
 *               values are clamped into [0, total_tokens] and a decreasing pair
 *               is treated as an empty sequence, so no access leaves the buffers
 *   scale       0 selects 1/sqrt(128)
 *   output      [total_tokens, 8, 128] bf16 (written, 8-byte aligned; rows outside every sequence untouched)
 *   new_state   [num_seqs, 8, 128, 128] fp32 (written; 16-byte aligned; must not be `state`)
 *   workspace   device scratch of at least gdn_prefill_workspace_min_bytes() bytes (normally
 *               gdn_prefill_workspace_bytes()), 256-byte aligned; workspace_bytes is its size
 *
 * Supported input domain (outputs within allclose(atol=1e-2, rtol=1e-2) of the
 * fp32 oracle and states within 2e-3 of its largest |state|): keys of any norm
 * and any beta = sigmoid(b) for which every token map g (I - beta k k^T) is a
 * contraction, i.e. |1 - beta |k|^2| <= 1 (L2-normalised keys with any b,
 * and for example |k|^2 = 1.5 with beta <= 0.8, are tested), with any gate
 * decay and any magnitude of v and of the state (tested from 1e-6 to 1e5, and
 * beta down to 2e-9).  The two fp16 operands of Delta = Tb (V - gam K S^T)
 * are scaled by powers of two into fp16's normal range before conversion.
 * Outside that domain the recurrence itself grows without bound and the
 * results are not specified.
 */
int gdn_prefill_fwd(const void* q, const void* k, const void* v, const float* state,
                    const float* A_log, const void* a, const float* dt_bias, const void* b,
                    const void* cu_seqlens, int cu_seqlens_is_int64, int num_seqs,
                    long long total_tokens, float scale, void* output, float* new_state,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Prefill that allocates nothing: gdn_prefill_fwd with its workspace taken from
 * a file-scope device array of GDN_PREFILL_NOALLOC_SCRATCH_BYTES (128 MiB),
 * which each GPU the library runs on holds until the process ends.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Arguments as gdn_prefill_fwd without the workspace;
 * `stream` must belong to the current device.  Returns GDN_ERR_TOO_LARGE when
 * gdn_prefill_workspace_min_bytes(num_seqs, total_tokens) exceeds the array
 * (about 145k tokens).  While the default workspace fits in the array (about
 * 28k tokens) results equal gdn_prefill_fwd's with a default workspace; beyond
 * that the planner has fewer segment slots and results stay within tolerance.  Every call on one GPU shares that
 * GPU's array: calls that overlap in time on one GPU (other streams, other host
 * threads) race and must be ordered by the caller.  Nothing in the array needs
 * to be cleared between calls.  The first call on each device resolves the
 * array's device address (which may load its code object): make that call
 * before capturing a HIP graph on the device; later calls, captured or not,
 * only launch kernels.  The array sits in its own code object, so processes
 * that never call this entry point do not hold it. */
int gdn_prefill_fwd_noalloc(const void* q, const void* k, const void* v, const float* state,
                            const float* A_log, const void* a, const float* dt_bias, const void* b,
                            const void* cu_seqlens, int cu_seqlens_is_int64, int num_seqs,
                            long long total_tokens, float scale, void* output, float* new_state,
                            void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GDN_MI355X_H */
