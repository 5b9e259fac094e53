/*
 * based_la.h -- C ABI of the MI355X (gfx950) BASED linear-attention library (libbased_la.so).
 *
 * Plain C: device pointers, sizes and a HIP stream handle, no C++ or torch types.  Every
 * tensor is a contiguous row-major (B, H, N, .) array in device memory owned by the caller;
 * the library allocates nothing per call.  Launches are asynchronous on the given stream
 * (NULL = the default stream); the caller synchronises.
 *
 * Return value: 0 on success; a negative LA_ERR_* code for an argument error detected on the
 * host before anything is launched; a positive value is a hipError_t reported by the runtime
 * right after the launch.  la_status_string() turns either into text.  Nothing throws.
 *
 * The entry points replace the reference's Python-level kernel wrappers
 * (Willy-Chan/trainium-linear-attention); each declaration names the function it stands in for.
 */
#ifndef BASED_LA_H
#define BASED_LA_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LA_ABI_VERSION 10

/* element types */
#define LA_F32 0
#define LA_BF16 1

/* argument errors (negative) */
#define LA_OK 0
#define LA_ERR_NULL_POINTER (-1)
#define LA_ERR_BAD_SHAPE (-2)
#define LA_ERR_BAD_DTYPE (-3)
#define LA_ERR_BAD_SCALAR (-4)
#define LA_ERR_UNSUPPORTED_DIM (-5)
#define LA_ERR_WORKSPACE (-6)
#define LA_ERR_NO_DEVICE (-7)
#define LA_ERR_BAD_ALIGNMENT (-8)
#define LA_ERR_OVERLAP (-9)
#define LA_ERR_SCRATCH_LIMIT (-10)

/* Size of the device array behind la_based_chunked_fwd_noalloc, per device. */
#define LA_NOALLOC_SCRATCH_BYTES (32u << 20)

/* Version of this ABI (LA_ABI_VERSION). */
int la_abi_version(void);

/* Static text for a status code returned by any la_* function. */
const char* la_status_string(int status);

/*
 * Fused causal BASED attention, parallel (quadratic) form.
 *
 * Replaces solution_nki / the NKI parallel kernel: kernels/pytorch_attention.py:44-78 and
 * kernels/nki_attention.py:25-115 (num and den accumulated per query block, out = num/(den+eps)).
 *
 *   s_tu = scale * q_t.k_u,  p = 1 + s + s^2/2,  den_t = sum_{u<=t} p_tu,
 *   num_t = sum_{u<=t} p_tu v_u,  out_t = normalize ? num_t / (den_t + eps) : num_t.
 *
 * q, k: (B,H,N,d); v, out: (B,H,N,dv); in_dtype / out_dtype: LA_BF16 or LA_F32 (q, k and v
 * share in_dtype).  den_or_null: optional (B,H,N) fp32 output of den_t (without eps).
 * workspace: device scratch of at least la_based_parallel_workspace_bytes(...) bytes, 16-byte
 * aligned (may be NULL when that is 0).  It holds V repacked as fp16 V^T blocks and prefix
 * sums over 64-key blocks of the column sums of V, of k and of k k^T for the bf16, d = 16,
 * dv % 8 == 0, dv <= 64 kernel; for fp32 inputs on small grids (2 to 255 query blocks of 128
 * tokens in all heads together) the partial numerators and row sums of every (query block,
 * pair of 64-key blocks), which a second kernel adds; its contents on return are unspecified.
 * Limits: 1 <= d <= 128, 1 <= dv <= 128, scale > 0 and finite, eps >= 0 and finite.
 * The reference passes scale = 1/sqrt(d) and eps = 1e-6.
 */
size_t la_based_parallel_workspace_bytes(int B, int H, int N, int d, int dv, int in_dtype);
int la_based_parallel_fwd(const void* q, const void* k, const void* v, int in_dtype,
                          void* out, int out_dtype, float* den_or_null,
                          int B, int H, int N, int d, int dv,
                          float scale, float eps, int normalize,
                          void* workspace, size_t workspace_bytes, void* hip_stream);

/*
 * The two halves of la_based_parallel_fwd for shapes that use the workspace: the K/V pre-pass,
 * and the attention kernel reading a workspace that already holds the pre-pass of the same k
 * and v (several calls with one k and v, or timing the attention kernel alone).  No counterpart in the
 * reference, whose parallel kernel has no pre-pass (kernels/nki_attention.py:33-115).  For
 * fp32 inputs and for shapes with la_based_parallel_workspace_bytes(...) == 0 the pack is a
 * no-op and la_based_parallel_fwd_packed is la_based_parallel_fwd.  The packed kernels need q, k, out
 * 16-byte and v 8-byte aligned (LA_ERR_BAD_ALIGNMENT otherwise; la_based_parallel_fwd instead
 * falls back to its unpacked kernel).
 */
int la_based_parallel_pack(const void* k, const void* v, int in_dtype, int B, int H, int N, int d, int dv,
                           void* workspace, size_t workspace_bytes, void* hip_stream);
int la_based_parallel_fwd_packed(const void* q, const void* k, const void* v, int in_dtype,
                                 void* out, int out_dtype, float* den_or_null,
                                 int B, int H, int N, int d, int dv,
                                 float scale, float eps, int normalize,
                                 void* workspace, size_t workspace_bytes, void* hip_stream);

/*
 * Chunked recurrent BASED attention (linear in N).
 *
 * Replaces chunked_nki_numerator / the NKI chunked kernel:
 * benchmarks/chunked_attention_benchmark.py:96-126 and kernels/nki_attention_chunked.py:20-113.
 * The feature map phi (benchmarks/chunked_attention_benchmark.py:34-53, dimension
 * F = 1 + d + d(d+1)/2) is applied inside the kernel; the (F x dv) state and the F-long K-sum
 * stay on chip across chunks.  normalize = 0 returns the numerator only (what the reference's
 * chunked kernel returns); normalize = 1 divides by phi(q).z + eps like the parallel path.
 * state_out_or_null: optional fp32 output of the final state per head, (B,H,F,dv+1) with the
 * K-sum in the last column.  workspace: device scratch of at least
 * la_based_chunked_workspace_bytes(...) bytes, 16-byte aligned (LA_ERR_BAD_ALIGNMENT otherwise;
 * may be NULL when that size is 0).
 * chunk: the reference's chunk_size, any value >= 1 (LA_ERR_BAD_SHAPE below 1).  The recurrence
 * computes the same function for every chunk size (chunk-size invariance); it runs in chunks of
 * la_based_chunked_chunk_used(chunk) tokens.
 * Limits: 1 <= d <= 64, 1 <= dv <= 128.  bf16 inputs with d == 16 and dv <= 64 run the chunk
 * recurrence (128-token chunks, state export and import); other shapes and fp32 inputs run the
 * segment-state path (state prefixes of 512-token segments in the feature basis, then each query
 * against its segment's prefix plus the quadratic form inside the segment; fp32 arithmetic
 * throughout for fp32 inputs), which has no state export here (LA_ERR_UNSUPPORTED_DIM with
 * state_out_or_null set): a caller continues such a sequence with la_based_chunked_fwd_num_den
 * and the state's contraction with phi(q) (the Python layer does this with
 * la_taylor_feature_map and fp32 GEMMs).  Both are linear in N.
 */
size_t la_based_chunked_workspace_bytes(int B, int H, int N, int d, int dv, int chunk);

/*
 * The same for one input type (LA_BF16 or LA_F32; (size_t)-1 for others): the scratch the
 * chunked entry points need for inputs of that type, which for fp32 inputs is the segment-state
 * path's fp32 state prefixes.  la_based_chunked_workspace_bytes returns the larger of the two.
 */
size_t la_based_chunked_workspace_bytes_dt(int B, int H, int N, int d, int dv, int chunk, int in_dtype);

/*
 * Tokens per chunk the chunked kernels run for a requested chunk size (128 for every chunk >= 1;
 * LA_ERR_BAD_SHAPE for chunk < 1).  The reference builds one NKI kernel per chunk_size
 * (kernels/nki_attention_chunked.py:20-30); here the kernel's chunk is fixed and reported.
 */
int la_based_chunked_chunk_used(int chunk);

int la_based_chunked_fwd(const void* q, const void* k, const void* v, int in_dtype,
                         void* out, int out_dtype, int B, int H, int N, int d, int dv, int chunk,
                         float scale, float eps, int normalize,
                         void* workspace, size_t workspace_bytes, float* state_out_or_null,
                         void* hip_stream);

/*
 * The two parts of the normalised output, separately: num_out (B,H,N,dv) fp32 the numerator
 * sum_{u<=t} p_tu v_u and den_out (B,H,N) fp32 the denominator sum_{u<=t} p_tu (no eps), for
 * callers that add terms of their own before dividing (e.g. an earlier segment's state applied
 * to these queries, out = (num + phi(q) S) / (den + phi(q) z + eps)).  Both must be 4-byte
 * aligned.  Every shape of la_based_chunked_fwd, with its workspace.  No reference counterpart
 * (the reference's chunked kernel returns the numerator only, kernels/nki_attention_chunked.py:56).
 */
int la_based_chunked_fwd_num_den(const void* q, const void* k, const void* v, int in_dtype,
                                 float* num_out, float* den_out, int B, int H, int N, int d, int dv,
                                 int chunk, float scale, void* workspace, size_t workspace_bytes,
                                 void* hip_stream);

/*
 * la_based_chunked_fwd continuing from an initial state: the sequence is the prev_tokens
 * tokens summarised by state_in followed by these N.  state_in: fp32 (B,H,F,dv+1) in the layout
 * of state_out (as exported by an earlier call, or updated by la_based_decode_step), not
 * overlapping state_out (LA_ERR_OVERLAP); prev_tokens: its token count (z[0], the same for every
 * head).  Output rows are tokens prev_tokens .. prev_tokens + N - 1 of the whole sequence;
 * state_out (optional) covers all prev_tokens + N.  No reference counterpart (the reference
 * starts every call from a zero state, kernels/nki_attention_chunked.py:66-69).
 */
int la_based_chunked_fwd_continue(const void* q, const void* k, const void* v, int in_dtype,
                                  void* out, int out_dtype, int B, int H, int N, int d, int dv,
                                  int chunk, float scale, float eps, int normalize,
                                  void* workspace, size_t workspace_bytes, const float* state_in,
                                  long long prev_tokens, float* state_out_or_null, void* hip_stream);

/*
 * la_based_chunked_fwd without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid allocation).
 * No counterpart in the reference.  The kernels' scratch is a fixed device array of
 * LA_NOALLOC_SCRATCH_BYTES inside the library (one per device, held until the process ends);
 * shapes that would need more return LA_ERR_SCRATCH_LIMIT before touching the device.  For bf16
 * d = 16, dv <= 64 (the chunk recurrence) 32 MiB covers every shape: at most about 1022 (head,
 * segment) records of 24 KiB are used.  The segment-state path (other d, dv > 64, fp32 inputs)
 * keeps state prefixes per (head, 512-token segment), which grow with B*H*N: e.g. bf16 B2 H16
 * N8192 d64 needs 224 MiB and is refused (la_based_chunked_workspace_bytes_dt gives the need).
 * The call allocates nothing.  Calls
 * that overlap in time on one device share the array and race: serialise them (one stream, or
 * the caller's own ordering).  Other arguments, limits and results as la_based_chunked_fwd.
 */
int la_based_chunked_fwd_noalloc(const void* q, const void* k, const void* v, int in_dtype,
                                 void* out, int out_dtype, int B, int H, int N, int d, int dv,
                                 int chunk, float scale, float eps, int normalize,
                                 float* state_out_or_null, void* hip_stream);

/*
 * Causal sliding-window softmax attention.
 *
 * Replaces nki_sliding_window_attn / the NKI sliding kernel:
 * benchmarks/sliding_attention_benchmark.py:59-99 and kernels/nki_attention_sliding.py:30-132
 * (valid keys t-W+1 <= u <= t, softmax of scale*q.k, times V).  Any window >= 1.
 * q, k: (B,H,N,d); v, out: (B,H,N,dv).  Limits: 1 <= d <= 128, 1 <= dv <= 128.
 */
int la_sliding_window_fwd(const void* q, const void* k, const void* v, int in_dtype,
                          void* out, int out_dtype, int B, int H, int N, int d, int dv,
                          int window, float scale, void* hip_stream);

/*
 * Sliding-window softmax attention plus an fp32 addend, out = sliding(q, k, v) + addend: the
 * second half of the full BASED layer, final = linear_attention + sliding_window_softmax
 * (kernels/nki_attention_sliding.py:4-5), with the linear-attention output as the addend.  The
 * sum is taken in fp32 in the sliding kernel's store, then rounded once to out_dtype.
 * addend: fp32 (B,H,N,dv), 16-byte aligned; it may be out itself when out_dtype is fp32.
 * Other arguments and limits as la_sliding_window_fwd.  (The reference computes the two
 * branches separately and has no entry point for the sum.)
 */
int la_sliding_window_fwd_add(const void* q, const void* k, const void* v, int in_dtype,
                              const float* addend, void* out, int out_dtype, int B, int H, int N,
                              int d, int dv, int window, float scale, void* hip_stream);

/*
 * The full BASED layer in one output launch: out = linear_attention(q, k, v) +
 * sliding_window_softmax(q_sw, k_sw, v) (kernels/nki_attention_sliding.py:4-5, whose two
 * branches the reference computes in separate calls; no single reference entry point).  The
 * linear branch is la_based_chunked_fwd's (scale, eps, normalised), the softmax branch
 * la_sliding_window_fwd's (scale_sw, window); after the chunked state passes one kernel computes
 * both branches per (head, segment) and stores their sum, rounded once to out_dtype.
 * q, k: (B,H,N,16); q_sw, k_sw: (B,H,N,d_sw); v, out: (B,H,N,dv); all bf16 inputs, every
 * tensor 16-byte aligned.  workspace: la_based_chunked_workspace_bytes_dt(B, H, N, 16, dv, 64,
 * LA_BF16) bytes, 16-byte aligned.  Limits: d = 16, dv % 8 == 0 and dv <= 64, d_sw in {16, 32, 64},
 * 1 <= window <= 64 (LA_ERR_UNSUPPORTED_DIM otherwise; such layers are the two calls).
 */
int la_based_layer_fwd(const void* q, const void* k, const void* v, const void* q_sw, const void* k_sw,
                       int in_dtype, void* out, int out_dtype, int B, int H, int N, int d, int dv, int d_sw,
                       int window, float scale, float scale_sw, float eps, void* workspace,
                       size_t workspace_bytes, void* hip_stream);

/*
 * One decode step of BASED attention on an exported state (no reference counterpart: the
 * reference has no decode path; this continues la_based_chunked_fwd's state_out).
 * state: fp32 (B,H,F,dv+1), F = 1 + d + d(d+1)/2, [S | z] in the feature order of
 * taylor_feature_map (benchmarks/chunked_attention_benchmark.py:34-53), updated in place with the
 * new token: [S | z] += phi(k) [v | 1].  Then out = phi(q)^T S / (phi(q)^T z + eps) with
 * normalize = 1 (the numerator phi(q)^T S with normalize = 0), which is the chunk recurrence of
 * kernels/nki_attention_chunked.py:65-109 for a chunk of one token.
 * q, k: (B,H,d) (one token per head); v, out: (B,H,dv).  Limits: 1 <= d <= 64, 1 <= dv <= 128.
 */
int la_based_decode_step(const void* q, const void* k, const void* v, int in_dtype,
                         float* state, void* out, int out_dtype, int B, int H, int d, int dv,
                         float eps, int normalize, void* hip_stream);

/*
 * la_based_decode_step with a caller-owned workspace (no reference counterpart, like
 * la_based_decode_step).  The workspace lets a small batch split every head's state rows over
 * several work-groups, whose partial column sums are then added in a fixed order
 * (deterministic, but rounded differently from la_based_decode_step).
 * la_based_decode_workspace_bytes gives the size.  It is 0 when a head's state fits in LDS
 * (F*(dv+1) <= 10240 floats), when one work-group per head already fills the device, or for
 * shapes outside the limits; the workspace can then be NULL, and the call is
 * la_based_decode_step.  Otherwise it holds B*H*R*(dv+1) floats for R row groups per
 * head.  It must be 4-byte aligned and must not overlap state, q, k, v or out.
 */
size_t la_based_decode_workspace_bytes(int B, int H, int d, int dv);
int la_based_decode_step_ws(const void* q, const void* k, const void* v, int in_dtype,
                            float* state, void* out, int out_dtype, int B, int H, int d, int dv,
                            float eps, int normalize, void* workspace, size_t workspace_bytes,
                            void* hip_stream);

/*
 * Causal linear attention with the identity feature map, numerator only:
 * out_t = sum_{u <= t} (scale q_t . k_u) v_u.
 *
 * Replaces ref_identity_numerator (benchmarks/chunked_attention_benchmark.py:81-93, scale
 * 1/sqrt(d)) and the chunked identity NKI kernel (old/identity_linear_attn_nki_CHUNKED.py:27-59,
 * whose state S = sum K^T V is carried here as exclusive prefixes over 64-token blocks).
 * q, k: (B,H,N,d) bf16; v, out: (B,H,N,dv); q, k, v, out 16-byte aligned.
 * workspace: device scratch of at least la_identity_workspace_bytes(...) bytes, 16-byte aligned.
 * Limits: bf16 inputs, d in {16, 32, 64}, dv in {32, 64} (la_identity_workspace_bytes returns 0
 * for other d, dv).
 */
size_t la_identity_workspace_bytes(int B, int H, int N, int d, int dv);
int la_identity_linear_fwd(const void* q, const void* k, const void* v, int in_dtype,
                           void* out, int out_dtype, int B, int H, int N, int d, int dv,
                           float scale, void* workspace, size_t workspace_bytes, void* hip_stream);

/*
 * BASED Taylor feature map, phi(x) = [1, x/d^(1/4), x_i^2/(sqrt(d) sqrt(2)),
 * x_i x_j/sqrt(d) (i<j, row-major upper-triangle order)], rows x (rows, d) -> (rows, F).
 *
 * Replaces taylor_feature_map: benchmarks/chunked_attention_benchmark.py:23-53.
 * Limits: 1 <= d <= 128.
 */
int la_taylor_feature_map(const void* x, int in_dtype, void* out, int out_dtype,
                          long long rows, int d, void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* BASED_LA_H */
