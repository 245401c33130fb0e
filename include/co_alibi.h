/*
 * co_alibi.h - C ABI of the MI355X (gfx950) Co-ALiBi attention library.
 *
 * The library holds the two hot-path launches of the reference
 * (Nathancgy/Co-ALIBI) behind plain pointers and sizes:
 *
 *   co_alibi_fwd  replaces the forward launch `_co_alibi_fwd_kernel[grid](...)`
 *                 in co_alibi_attn/co_alibi_attn.py:41-57 (and the O / LSE /
 *                 RowSigTotal allocations at :35-37 move to the caller).
 *   co_alibi_bwd  replaces the backward launch `_co_alibi_bwd_kernel[grid](...)`
 *                 in co_alibi_attn/co_alibi_attn.py:101-123 together with the
 *                 dK/dV partial buffers and their reduction (:83-99, :132-133).
 *
 * and a decode step the reference does not have, co_alibi_decode: its forward
 * with Sq = 1 over a key / value cache, as one split-K pass over the cache.
 *
 * Tensor layout: contiguous row-major, q / o / dout / dq are (B, Hq, Sq, D),
 * k / v / dk / dv are (B, Hkv, Skv, D); query head h attends key/value head
 * h / (Hq / Hkv) (the head mapping of co_alibi_attn.py:143-146, done in-kernel
 * instead of by repeat_interleave).  Element type is selected by `dtype`; all
 * statistics are fp32.  `slopes` holds Hq fp32 penalty slopes (the caller
 * rounds them to the input dtype first, as co_alibi_attn.py:147 does).
 * Causal masking is top-left aligned (key j is visible to query i iff j <= i).
 *
 * Every call is asynchronous on `stream` (a hipStream_t; NULL = the null
 * stream), allocates nothing, and returns CO_ALIBI_OK or an error code; the
 * message of the last failure on the calling thread is co_alibi_last_error().
 * Pointers to element data must be 16-byte aligned, fp32 arrays 4-byte aligned.
 * Head dims 16, 32, 64, 128 and 256 in every dtype (the decode: 32 to 256, and 256 only
 * in fp16 / bf16).
 */
#ifndef CO_ALIBI_H
#define CO_ALIBI_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum co_alibi_dtype { CO_ALIBI_F32 = 0, CO_ALIBI_F16 = 1, CO_ALIBI_BF16 = 2 };

enum co_alibi_status {
  CO_ALIBI_OK = 0,
  CO_ALIBI_EINVAL = 1,       /* bad pointer, size, alignment or workspace */
  CO_ALIBI_EUNSUPPORTED = 2, /* dtype or head_dim without a kernel */
  CO_ALIBI_ELAUNCH = 3       /* the HIP runtime refused the launch */
};

/* Number of 4-byte words of the statistics `stats` that co_alibi_fwd writes beside lse and
 * co_alibi_bwd reads: 4 + B*Hq * (2 * ceil(Sq/128) + ceil(Skv/256) + ceil(Skv/64) + 2 * Sq),
 * O(B*Hq*S).  A 4-word header (flags: which work orders the forward wrote); per 128-row block
 * the first key the forward processed (int32; keys further left carry softmax weights below
 * 2^-T of their row's total, T = 26 in fp16, 32 in bf16 and 64 in fp32, and are skipped by
 * forward and backward alike; 0 when the tail skip is off); per 256-key chunk of each key head
 * the largest |k|; the order in which the kernels take their row and key blocks (int32); and
 * per row the sum of the sigmoids of the processed keys, as an fp32 hi part (B*Hq*Sq) and its
 * compensation (B*Hq*Sq).  That row sum is the reference's RowSigTotal (co_alibi_attn.py:37);
 * the backward rebuilds the penalty from it. */
size_t co_alibi_stats_numel(int batch, int heads_q, int seq_q, int seq_kv);

/* The tail skip as a library setting, for every later co_alibi_fwd and co_alibi_fwd_inference
 * call of the process: enabled != 0 (the default) leaves out the keys whose softmax weight is
 * provably below 2^-T of their row's total (above), 0 makes the forward process every key, as
 * the reference does (co_alibi_fwd_kernel.py:66-71), with no key-norm launch and no per-tile
 * test.  The backward follows what its forward recorded.  Returns the previous setting.  No
 * counterpart in the reference, which processes every key. */
int co_alibi_set_tail_skip(int enabled);
int co_alibi_tail_skip(void);

/* Bytes of device scratch co_alibi_bwd needs (the recompute path): per-row dO.O, then per 32-key
 * block of every row the sigmoid sum from the block start on and the dA sum before it,
 * 2 * B*Hq * ceil(Skv/32) * Sq fp32 -- transient, the backward's own, where the reference holds
 * its per-query-block dK / dV partials (co_alibi_attn.py:83-99). */
size_t co_alibi_bwd_workspace_bytes(int batch, int heads_q, int seq_q, int seq_kv);

/* Bytes of device scratch that switch the backward to the score store: pass 1 keeps the
 * probabilities and score gradients of every tile it processes, 4 KB per 32 x 32 block of
 * pairs that can be visible (about 2 * Sq * Skv bytes per batch and query head when causal,
 * twice that otherwise), and pass 2 reduces them into dk and dv instead of recomputing
 * them.  0 when dtype / head_dim have no such path (fp16 and bf16 at head_dim 64 and 128
 * have it) or when (heads_q / heads_kv) * ceil(seq_q / 8192) exceeds 256.  A workspace of at
 * least this size selects the path; a smaller one (at least
 * co_alibi_bwd_workspace_bytes) the recompute path.  co_alibi_bwd_dq and co_alibi_bwd_dkdv
 * must then get the same workspace and size.  No counterpart in the reference, whose
 * backward keeps per-query-block dK / dV partials instead (co_alibi_attn.py:83-133). */
size_t co_alibi_bwd_score_store_workspace_bytes(int dtype, int batch, int heads_q, int heads_kv, int seq_q,
                                                int seq_kv, int head_dim, int causal);

/* Forward: writes o (B,Hq,Sq,D, dtype), lse (B,Hq,Sq, fp32 natural log-sum-exp
 * m_i + log(l_i), co_alibi_fwd_kernel.py:120) and stats.  The reference adds 1e-9
 * to l_i there and in the O normaliser (:115); l_i >= 1 here, so that term is
 * below fp32 resolution and is left out.  lse and stats may be NULL (inference: the
 * statistics only co_alibi_bwd reads are then not written, and every key is
 * processed); o is the same. */
int co_alibi_fwd(int dtype, const void* q, const void* k, const void* v, const float* slopes,
                 void* o, float* lse, float* stats, int batch, int heads_q, int heads_kv, int seq_q,
                 int seq_kv, int head_dim, int causal, float sm_scale, void* stream);

/* Forward for inference with the tail skip: o only (no lse or stats), skipping the keys
 * whose softmax weight is below 2^-T of the row total as co_alibi_fwd does with its
 * statistics (co_alibi_fwd with lse = stats = NULL computes every key).  workspace holds
 * co_alibi_fwd_inference_workspace_bytes(...) bytes (256-byte aligned): the largest |k|
 * per 256-key chunk of every key head and the order of the row blocks.  No counterpart in
 * the reference, whose forward always saves its statistics (co_alibi_attn.py:35-57). */
size_t co_alibi_fwd_inference_workspace_bytes(int batch, int heads_q, int seq_q, int seq_kv);
int co_alibi_fwd_inference(int dtype, const void* q, const void* k, const void* v, const float* slopes,
                           void* o, void* workspace, size_t workspace_bytes, int batch, int heads_q,
                           int heads_kv, int seq_q, int seq_kv, int head_dim, int causal, float sm_scale,
                           void* stream);

/* Backward: given dout and the forward's q, k, v, o, lse, stats, writes dq
 * (B,Hq,Sq,D), dk and dv (B,Hkv,Skv,D), all in dtype.  For Hkv < Hq the key /
 * value gradients are summed over the query heads of each group.  workspace
 * must hold co_alibi_bwd_workspace_bytes(...) bytes (256-byte aligned). */
int co_alibi_bwd(int dtype, const void* dout, const void* q, const void* k, const void* v,
                 const void* o, const float* lse, const float* stats, const float* slopes, void* dq,
                 void* dk, void* dv, void* workspace, size_t workspace_bytes, int batch, int heads_q,
                 int heads_kv, int seq_q, int seq_kv, int head_dim, int causal, float sm_scale,
                 void* stream);

/* The two passes of co_alibi_bwd as separate calls, for callers that time or
 * schedule them apart.  co_alibi_bwd_dq writes dq and fills the workspace
 * (per-row dO.O and the per-32-key-block sums, or the score store); co_alibi_bwd_dkdv
 * then writes dk and dv from that workspace.  Issued in this order on one
 * stream they are exactly co_alibi_bwd.  The reference runs both in one
 * kernel (co_alibi_attn/co_alibi_bwd_kernel.py:17-146). */
int co_alibi_bwd_dq(int dtype, const void* dout, const void* q, const void* k, const void* v,
                    const void* o, const float* lse, const float* stats, const float* slopes, void* dq,
                    void* workspace, size_t workspace_bytes, int batch, int heads_q, int heads_kv,
                    int seq_q, int seq_kv, int head_dim, int causal, float sm_scale, void* stream);

int co_alibi_bwd_dkdv(int dtype, const void* dout, const void* q, const void* k, const void* v,
                      const float* lse, const float* stats, const float* slopes, void* dk, void* dv,
                      void* workspace, size_t workspace_bytes, int batch, int heads_q, int heads_kv,
                      int seq_q, int seq_kv, int head_dim, int causal, float sm_scale, void* stream);

/* Bytes of device scratch co_alibi_decode needs: the split-K partials, 4 + head_dim
 * fp32 per (batch, query head, split), for min(ceil(seq_kv / 128), 1024) splits (each
 * split walks one or more 128-key chunks of the cache). */
size_t co_alibi_decode_workspace_bytes(int batch, int heads_q, int seq_kv, int head_dim);

/* Decode: one new query per (batch, query head) against a key / value cache.
 * q and o are (B, Hq, D); k_cache and v_cache are (B, Hkv, kv_capacity, D).  Sequence
 * b has its first len_b rows of every head filled, all of them visible to the query
 * (the newest position): len_b = seq_lens[b] when seq_lens (B int32 on the device) is
 * given, clamped to [0, seq_kv] in the kernel, else seq_kv.  A sequence of length 0
 * gets O = 0 and LSE = -inf.  lse (B*Hq fp32, natural log) may be NULL.  The
 * reference has no decode entry point: this is its forward, co_alibi_attention(q, k,
 * v, causal=False) (co_alibi_attn/co_alibi_attn.py:137-148), with Sq = 1 and the
 * caches cut to len_b rows; its top-left causal mask (co_alibi_fwd_kernel.py:80-90)
 * would show an Sq = 1 query only the first key.  Head dims 32 to 256 (256 in fp16 /
 * bf16 only); at most 32 query heads per kv head, seq_kv <= 2^21 (it sizes the grid and the workspace); workspace holds
 * co_alibi_decode_workspace_bytes(...) bytes (256-byte aligned). */
int co_alibi_decode(int dtype, const void* q, const void* k_cache, const void* v_cache,
                    const float* slopes, const int* seq_lens, void* o, float* lse,
                    void* workspace, size_t workspace_bytes, int batch, int heads_q, int heads_kv,
                    int seq_kv, int kv_capacity, int head_dim, float sm_scale, void* stream);

/* co_alibi_decode for callers that cannot allocate device memory (work captured into a HIP
 * graph, tight serving loops, harnesses that forbid hipMalloc).  It has no counterpart in the
 * reference.  Arguments are those of co_alibi_decode without the workspace: the split-K
 * partials go to a buffer of CO_ALIBI_DECODE_SCRATCH_BYTES that the library holds on every GPU
 * it runs on until the process ends, laid out for this launch's split count ((4 + head_dim)
 * fp32 per (batch, query head, split), each of the three per-split arrays 256-byte aligned).  A
 * decode whose partials exceed it returns CO_ALIBI_EINVAL.  The call allocates nothing.  All
 * calls on one GPU share its buffer, which keeps the last call's contents: calls that overlap on
 * one GPU (for instance on two streams) race, so order them on one stream. */
#define CO_ALIBI_DECODE_SCRATCH_BYTES (32u << 20)
int co_alibi_decode_noalloc(int dtype, const void* q, const void* k_cache, const void* v_cache,
                            const float* slopes, const int* seq_lens, void* o, float* lse, int batch,
                            int heads_q, int heads_kv, int seq_kv, int kv_capacity, int head_dim,
                            float sm_scale, void* stream);

/* Measurement helper with no counterpart in the reference: `blocks` work-groups of 256
 * threads each issue `iters` rounds of four independent fp16 32x32x16 MFMAs per
 * wavefront.  ticks (2*blocks uint64) receives, per work-group, the shader-clock and the
 * 100 MHz real-time counter deltas around the loop; sink (256*blocks fp32) receives a
 * checksum.  The benchmark derives the sustained clock and MFMA rate from it. */
int co_alibi_probe_mfma(void* ticks, void* sink, int blocks, int iters, void* stream);

/* Message describing the last failed call on this thread ("" if none). */
const char* co_alibi_last_error(void);

/* ABI version of this header: 6 (O(S) statistics, the row sigmoid sums in place of the
 * per-block penalty sums; the tail-skip setting). */
int co_alibi_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* CO_ALIBI_H */
