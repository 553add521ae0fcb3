/*
 * mykfa — MI355X (gfx950) FlashAttention, C ABI.
 *
 * This library is the native side of the drop-in replacement for the Triton kernels in
 * myk-llm's src/myk_llm/ops/flash_attn.py. Every entry point takes plain C structs of
 * device pointers, element strides and ints, launches asynchronously on the caller's
 * stream, never allocates or frees device memory, never synchronizes, and never throws or
 * aborts across the ABI: it returns a status code and leaves a message readable through
 * mykfa_last_error() on the calling thread.
 *
 * Semantics shared by every entry point (reference: flash_attn.py:11-22):
 *   - queries are aligned to the END of the keys: query i of a sequence with Lq queries and
 *     Lk keys sits at key position i + Lk - Lq and sees keys j with
 *         i + Lk - Lq - window_left  <=  j  <=  i + Lk - Lq + window_right,   0 <= j < Lk;
 *     a window side given as MYKFA_UNBOUNDED (2^30) is unbounded; causal is window_right=0
 *     (reference: _window, flash_attn.py:435-439);
 *   - GQA: query head h reads key/value head h / (num_heads / num_kv_heads)
 *     (flash_attn.py:122);
 *   - lse is the base-2 log-sum-exp of the scaled scores, fp32, laid out (num_heads, rows)
 *     with rows = total packed tokens (varlen) or batch * seqlen_q (dense); a row that sees
 *     no key gets lse = +inf and an output of 0 (flash_attn.py:147-153);
 *   - strides are in ELEMENTS, as (batch, token, head); the last dimension must be
 *     contiguous; batch stride 0 for packed varlen tensors (flash_attn.py:331-333).
 */
#ifndef MYKFA_H
#define MYKFA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MYKFA_ABI_VERSION 7
#define MYKFA_UNBOUNDED (1 << 30) /* flash_attn.py:32 (_UNBOUNDED) */

/* Status codes. */
#define MYKFA_OK 0
#define MYKFA_ERR_INVALID 1     /* malformed arguments (null pointer, bad stride, shape) */
#define MYKFA_ERR_UNSUPPORTED 2 /* valid but not implemented (head_dim, dtype) */
#define MYKFA_ERR_LAUNCH 3      /* the HIP runtime rejected a launch */
#define MYKFA_ERR_WORKSPACE 4   /* caller-provided workspace too small */

/* Element types of q/k/v/o (reference accepts bf16 and fp16: flash_attn.py:340-341). */
#define MYKFA_BF16 0
#define MYKFA_FP16 1

/* hipStream_t, without requiring the HIP headers in FFI users. NULL = default stream. */
typedef struct ihipStream_t* mykfa_stream_t;

/*
 * Forward parameters. Replaces the argument list of _forward / _fwd_kernel
 * (flash_attn.py:353-373, :106-114).
 *   dense  : cu_seqlens_q == cu_seqlens_k == NULL, q (batch, seqlen_q, H, D),
 *            k/v (batch, seqlen_k, Hkv, D); seqused_k (batch,) optionally limits each
 *            sequence's keys (the KV-cache path, flash_attn.py:486-488).
 *   varlen : cu_seqlens_q/k int32 (batch + 1,), packed q (total_q, H, D),
 *            k/v (total_k, Hkv, D); max_seqlen_q/k bound the per-sequence lengths.
 */
typedef struct mykfa_fwd_params {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;
    int64_t q_batch_stride, q_token_stride, q_head_stride;
    int64_t k_batch_stride, k_token_stride, k_head_stride;
    int64_t v_batch_stride, v_token_stride, v_head_stride;
    int64_t o_batch_stride, o_token_stride, o_head_stride;
    int64_t lse_head_stride; /* = rows: dense batch * max_seqlen_q; packed: at least the packed
                              * row count cu_seqlens_q[batch] (which only the device holds: a
                              * smaller stride is not detected, and the stored-dS backward then
                              * leaves the dQ rows beyond it unwritten) */
    const int32_t* cu_seqlens_q;
    const int32_t* cu_seqlens_k;
    const int32_t* seqused_k;
    int32_t batch;
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t max_seqlen_q; /* dense: seqlen_q */
    int32_t max_seqlen_k; /* dense: seqlen_k (cache capacity on the KV-cache path) */
    int32_t window_left;  /* >= 0; MYKFA_UNBOUNDED for none */
    int32_t window_right; /* >= 0; 0 when causal */
    float softmax_scale;
    int32_t dtype; /* MYKFA_BF16 / MYKFA_FP16 */
} mykfa_fwd_params;

/*
 * Backward parameters. Replaces the argument list of _backward / _bwd_dq_kernel /
 * _bwd_dkdv_kernel (flash_attn.py:376-406, :181-190, :264-273). The forward fields
 * (q, k, v, o, lse, sequence layout, window, scale) must be those of the forward call.
 * delta is an fp32 (num_heads, rows) buffer laid out like lse.
 */
typedef struct mykfa_bwd_params {
    mykfa_fwd_params fwd;
    const void* dout;
    void* dq;
    void* dk;
    void* dv;
    float* delta;
    int64_t do_batch_stride, do_token_stride, do_head_stride;
    int64_t dq_batch_stride, dq_token_stride, dq_head_stride;
    int64_t dk_batch_stride, dk_token_stride, dk_head_stride;
    int64_t dv_batch_stride, dv_token_stride, dv_head_stride;
} mykfa_bwd_params;

/*
 * KV-cache decode parameters (flash_attn_with_kvcache, flash_attn.py:467-490, run as a
 * split-K forward). q (batch, seqlen_q, H, D); caches (batch, capacity, Hkv, D) with a
 * contiguous last dimension; the keys of sequence b are cache rows
 * [0, seqused_k[b] + seqlen_new), clamped to [0, capacity] (all capacity rows when seqused_k
 * is NULL, which requires seqlen_new = 0).
 * New keys of this step (flash_attn_with_kvcache's k, v; flash_attn.py:480-485): with k_new
 * and v_new non-NULL the decode itself first writes them into the caches at rows
 * seqused_k[b] + t, t < seqlen_new (rows at or beyond the capacity are dropped), so fwd.k and
 * fwd.v are written through; with both NULL the seqlen_new rows must already be there
 * (mykfa_kv_append).
 * Partial results of each split go to a caller-provided workspace
 * (mykfa_decode_workspace_size) and are combined by an LSE merge.
 */
typedef struct mykfa_decode_params {
    mykfa_fwd_params fwd;   /* cu_seqlens_* must be NULL; seqused_k NULL = max_seqlen_k keys */
    int32_t num_splits;     /* partial slots per sequence on average (the workspace's segment
                             * pool is num_splits * batch); the kernel splits each sequence by
                             * its actual length within that pool. 1 = one split per sequence,
                             * no merge; 0 = choose (mykfa_decode_num_splits) */
    int32_t seqlen_new;     /* new keys per sequence after seqused_k[b] (0 = none) */
    const void* k_new;      /* (batch, seqlen_new, Hkv, D) or NULL */
    const void* v_new;
    int64_t kn_batch_stride, kn_token_stride, kn_head_stride;
    int64_t vn_batch_stride, vn_token_stride, vn_head_stride;
} mykfa_decode_params;

/* KV append: cache[b, cache_seqlens[b] + t] = new[b, t] for t < seqlen_new
 * (flash_attn.py:480-485). */
typedef struct mykfa_kv_append_params {
    void* k_cache;
    void* v_cache;
    const void* k_new;
    const void* v_new;
    const int32_t* cache_seqlens;
    int64_t kc_batch_stride, kc_token_stride, kc_head_stride;
    int64_t vc_batch_stride, vc_token_stride, vc_head_stride;
    int64_t kn_batch_stride, kn_token_stride, kn_head_stride;
    int64_t vn_batch_stride, vn_token_stride, vn_head_stride;
    int32_t batch;
    int32_t seqlen_new;
    int32_t capacity;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t dtype;
} mykfa_kv_append_params;

/*
 * Attention-block prologue: q/k RMSNorm (cast back to the input type) followed by the
 * interleaved-pair rotary embedding, in one pass over q and k. Replaces, in one launch, the
 * elementwise chain of Attention.forward (mixers.py:85-89): RMSNorm.forward
 * (model/layers.py:22-25) under bf16 autocast, `.to(v.dtype)`, then RotaryEmbedding.rotate
 * (model/layers.py:93-98) in fp32 and the cast back.
 *   q_in/k_in  (batch, seqlen, H, D) views, e.g. of the fused qkv projection output;
 *   q_out/k_out written in the input type;
 *   position_ids int64 (batch, seqlen) (batch stride 0 for an expanded arange); a position
 *   outside [0, table_rows) reads the nearest table row;
 *   cos/sin fp32 (table_rows, D): RotaryEmbedding.cos_cached / sin_cached (angles repeated
 *   per pair, layers.py:80-85); both NULL = no rotation;
 *   q_weight/k_weight fp32 (D,): the RMSNorm weights; both NULL = no norm.
 * Rounding points follow the reference under autocast: the norm in fp32, rounded to the
 * input type; the rotation in fp32 (separate products and sum, no fused multiply-add),
 * rounded to the input type.
 */
typedef struct mykfa_qk_prologue_params {
    const void* q_in;
    const void* k_in;
    void* q_out;
    void* k_out;
    int64_t qi_batch_stride, qi_token_stride, qi_head_stride;
    int64_t ki_batch_stride, ki_token_stride, ki_head_stride;
    int64_t qo_batch_stride, qo_token_stride, qo_head_stride;
    int64_t ko_batch_stride, ko_token_stride, ko_head_stride;
    const int64_t* position_ids;
    int64_t pos_batch_stride, pos_token_stride;
    const float* cos;
    const float* sin;
    int64_t table_stride; /* elements between table rows (>= head_dim, multiple of 4) */
    int32_t table_rows;
    const float* q_weight;
    const float* k_weight;
    float eps;
    int32_t batch;
    int32_t seqlen;
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t dtype;
} mykfa_qk_prologue_params;

/*
 * Prologue backward: gradients of q_in/k_in from those of q_out/k_out (autograd of the
 * forward chain above), the RMSNorm weight gradients summed over every token and head in a
 * fixed order (deterministic), and optionally a copy of the value gradient dv_src into dv_dst
 * so that one launch fills a whole fused-projection gradient (q | k | v slices).
 * fwd.q_in/k_in/positions/tables/weights/eps must be those of the forward call; fwd.q_out and
 * fwd.k_out are ignored. dq_weight/dk_weight (fp32 (D,)) are written, not accumulated, and are
 * required exactly when the forward had weights.
 */
typedef struct mykfa_qk_prologue_bwd_params {
    mykfa_qk_prologue_params fwd;
    const void* dq_out;
    const void* dk_out;
    void* dq_in;
    void* dk_in;
    int64_t dqo_batch_stride, dqo_token_stride, dqo_head_stride;
    int64_t dko_batch_stride, dko_token_stride, dko_head_stride;
    int64_t dqi_batch_stride, dqi_token_stride, dqi_head_stride;
    int64_t dki_batch_stride, dki_token_stride, dki_head_stride;
    const void* dv_src; /* (batch, seqlen, Hkv, D) or NULL */
    void* dv_dst;
    int64_t dvs_batch_stride, dvs_token_stride, dvs_head_stride;
    int64_t dvd_batch_stride, dvd_token_stride, dvd_head_stride;
    float* dq_weight;
    float* dk_weight;
} mykfa_qk_prologue_bwd_params;

/*
 * Attention-block epilogue: the output gate y = x * sigmoid(gate) (mixers.py:116-117) over
 * rows of `width` elements, with the reference's autocast rounding points (sigmoid rounded to
 * the input type, then the product rounded). Backward: dx = dy * s, and
 * dgate = (dy * x rounded) * (1 - s) * s, s = the rounded sigmoid (torch's mul and
 * sigmoid_backward). Row strides in elements; width a multiple of 8.
 */
typedef struct mykfa_gate_params {
    const void* x;
    const void* gate;
    void* y;       /* forward output */
    const void* dy; /* backward inputs/outputs (unused by the forward) */
    void* dx;
    void* dgate;
    int64_t x_row_stride, gate_row_stride, y_row_stride;
    int64_t dy_row_stride, dx_row_stride, dgate_row_stride;
    int64_t rows;
    int32_t width;
    int32_t dtype;
} mykfa_gate_params;

/*
 * Cross-entropy rows of the fused linear + cross-entropy (replaces _ce_kernel,
 * ops/fused_ce.py:20-67). For each row r of `logits` (a chunk of hidden @ weight^T):
 *   lse[r] = logsumexp(logits[r]),  ce[r] = lse[r] - logits[r, targets[r]]   (fp32), and
 *   logits[r] overwritten with softmax(logits[r]) * scale * (1 + 2 z_coef lse[r])
 *                                 - scale * onehot(targets[r])   (the gradient of
 *   scale * (ce + z_coef * lse^2) with respect to the logits);
 * rows whose target equals ignore_index get zeros and ce = lse = 0. A target outside
 * [0, vocab) other than ignore_index gives ce = NaN (no class to subtract).
 * targets are int64; the row stride is in elements.
 */
typedef struct mykfa_ce_params {
    void* logits;
    const int64_t* targets;
    float* ce;
    float* lse;
    int64_t row_stride;
    int64_t rows;
    int32_t vocab;
    int32_t ignore_index;
    float scale;
    float z_coef;
    int32_t dtype;
} mykfa_ce_params;

/*
 * Batched symmetric rank-K product of Muon's Newton-Schulz iteration (replaces
 * _batched_syrk_kernel, ops/muon.py:28-104):
 *   out[b] = alpha * x[b] x[b]^T + beta * bias[b]     x (batch, m, k), out (batch, m, m), bf16;
 * the lower-triangular tiles are computed and mirrored into the upper triangle (bias is read
 * at the computed positions, so it must be symmetric for a symmetric result, as in the
 * reference). Row strides in elements; k must be a multiple of 64 (callers pad with zero
 * columns); x 16-byte aligned with a row stride that is a multiple of 8; out 8-byte aligned
 * with a row stride that is a multiple of 4; bias NULL for none.
 */
typedef struct mykfa_syrk_params {
    const void* x;
    const void* bias;
    void* out;
    int64_t x_batch_stride, x_row_stride;
    int64_t bias_batch_stride, bias_row_stride;
    int64_t out_batch_stride, out_row_stride;
    int32_t batch;
    int32_t m;
    int32_t k;
    float alpha;
    float beta;
    int32_t dtype; /* MYKFA_BF16 */
} mykfa_syrk_params;

/* ---- version / errors ------------------------------------------------------------- */
int mykfa_abi_version(void);
const char* mykfa_version(void);
/* Message of the last failing call on this thread ("" if none). */
const char* mykfa_last_error(void);
/* sizeof() of each parameter struct, so bindings can check their mirror. */
size_t mykfa_sizeof_fwd_params(void);
size_t mykfa_sizeof_bwd_params(void);
size_t mykfa_sizeof_decode_params(void);
size_t mykfa_sizeof_kv_append_params(void);

/* ---- host-only validation (no GPU needed) ------------------------------------------ */
/* Checks of _check (flash_attn.py:336-346) plus pointer/stride/window sanity. */
int mykfa_validate_fwd(const mykfa_fwd_params* p);
int mykfa_validate_bwd(const mykfa_bwd_params* p);
int mykfa_validate_decode(const mykfa_decode_params* p);
int mykfa_validate_kv_append(const mykfa_kv_append_params* p);

/* ---- forward ----------------------------------------------------------------------- */
/* O and LSE (replaces _forward + _fwd_kernel, flash_attn.py:353-373, :106-154). */
int mykfa_fwd(const mykfa_fwd_params* p, mykfa_stream_t stream);

/* ---- backward ---------------------------------------------------------------------- */
/* delta = rowsum(dO * O) in fp32 (the preprocess fused into _bwd_dq_kernel,
 * flash_attn.py:215-216). */
int mykfa_bwd_preprocess(const mykfa_bwd_params* p, mykfa_stream_t stream);
/* dK, dV summed over each GQA group (replaces _bwd_dkdv_kernel, flash_attn.py:264-314).
 * Reads delta: run mykfa_bwd_preprocess or mykfa_bwd_dq first on the same stream. */
int mykfa_bwd_dkdv(const mykfa_bwd_params* p, mykfa_stream_t stream);
/* dQ (replaces _bwd_dq_kernel, flash_attn.py:181-230, with its fused delta preprocess,
 * :215-216): computes delta = rowsum(dO * O) itself and writes it to p->delta. */
int mykfa_bwd_dq(const mykfa_bwd_params* p, mykfa_stream_t stream);
/* dQ (with delta) then dK/dV in stream order (replaces _backward, flash_attn.py:376-406). */
int mykfa_bwd(const mykfa_bwd_params* p, mykfa_stream_t stream);
/* Backward through stored dS (replaces _backward, flash_attn.py:376-406, like mykfa_bwd):
 * delta, then dK/dV, which also stores every 32 x 32 block of dS (rounded to the input type,
 * as the reference rounds it before its dQ product, flash_attn.py:177) into the workspace,
 * then dQ = scale * dS K from those blocks: five products per (query tile, key block) pair
 * instead of seven. Deterministic: no sum depends on the order of workgroups (dK/dV takes its
 * blocks from queues through atomic counters, which decide only which workgroup computes a
 * block). The workspace holds the dS of whole KV heads (each query tile's row holds exactly
 * the key blocks its band touches), the queue counters and, for packed batches, a table of
 * sequence starts built on the device: mykfa_bwd_workspace_per_kv_head bytes per KV head (0 when
 * head_dim is not 128, where the trade does not pay; for packed batches an upper bound over all
 * length distributions with the given rows, batch and max_seqlen); with workspace_bytes >= n
 * times that, KV heads are processed in passes of up to n, with identical results for every n.
 * With less than one KV head's worth this is mykfa_bwd (dQ recomputes S and dP). The workspace
 * must be 16-byte aligned (MYKFA_ERR_INVALID otherwise); its contents on entry do not matter. */
size_t mykfa_bwd_workspace_per_kv_head(const mykfa_bwd_params* p);
int mykfa_bwd_ws(const mykfa_bwd_params* p, void* workspace, size_t workspace_bytes, mykfa_stream_t stream);
/* The two halves of mykfa_bwd_ws over every KV head in one launch each (workspace of
 * num_kv_heads * mykfa_bwd_workspace_per_kv_head bytes, else MYKFA_ERR_WORKSPACE):
 * dK/dV storing dS (replaces _bwd_dkdv_kernel, flash_attn.py:264-314; reads delta, so run
 * mykfa_bwd_preprocess first), then dQ from the stored dS (replaces _bwd_dq_kernel,
 * flash_attn.py:181-230, without its S / dP recompute). */
int mykfa_bwd_dkdv_ws(const mykfa_bwd_params* p, void* workspace, size_t workspace_bytes, mykfa_stream_t stream);
int mykfa_bwd_dq_ws(const mykfa_bwd_params* p, void* workspace, size_t workspace_bytes, mykfa_stream_t stream);

/* ---- KV-cache decode (split-K) ------------------------------------------------------ */
/* Slots per sequence the library would pick for this shape (>= 1): about 1400 keys of capacity
 * per slot, enough to fill the chip (the query rows per KV head set how many workgroups a split
 * has), at least 128 keys per slot. The split-K pass itself sizes its splits from the actual
 * lengths on the device (so that its active workgroups fit one resident round of the chip) and
 * uses at most num_splits * batch segments. */
int mykfa_decode_num_splits(int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t seqlen_q,
                            int32_t capacity);
/* Bytes of workspace mykfa_decode needs for this shape and split count. */
size_t mykfa_decode_workspace_size(int32_t batch, int32_t num_heads, int32_t seqlen_q,
                                   int32_t head_dim, int32_t num_splits);
/* Split-K partial pass: writes per-split (O, LSE) into the workspace. */
int mykfa_decode_splitk(const mykfa_decode_params* p, void* workspace, size_t workspace_bytes,
                        mykfa_stream_t stream);
/* LSE merge of the per-split partials into o and lse. */
int mykfa_decode_merge(const mykfa_decode_params* p, const void* workspace,
                       size_t workspace_bytes, mykfa_stream_t stream);
/* split-K + merge (replaces _forward's decode configuration, flash_attn.py:364, :488, and,
 * with k_new / v_new, the cache writes of flash_attn_with_kvcache, flash_attn.py:480-485). */
int mykfa_decode(const mykfa_decode_params* p, void* workspace, size_t workspace_bytes,
                 mykfa_stream_t stream);

/* Size of the static scratch array behind mykfa_decode_noalloc (per GPU, held until the
 * process ends). */
#define MYKFA_DECODE_SCRATCH_BYTES ((size_t)16 << 20)
/* Allocation-free split-K decode + merge: no counterpart in the reference. For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). Same parameters and results as mykfa_decode, but the split partials
 * live in a file-scope device array of MYKFA_DECODE_SCRATCH_BYTES (16 MiB) instead of a
 * caller workspace; nothing is allocated or freed. With num_splits = 0 the library's split
 * count is cut to what the scratch holds; an explicit num_splits whose partials exceed it is
 * rejected (MYKFA_ERR_WORKSPACE). Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (concurrent streams) race and must be serialized by the caller. Nothing
 * in the array needs to start at zero (each call writes every partial its merge reads). The
 * first call on each device (the device of `stream`, whichever device is current) resolves the
 * array's address (hipGetSymbolAddress): make one call outside graph capture before capturing. */
int mykfa_decode_noalloc(const mykfa_decode_params* p, mykfa_stream_t stream);

/* ---- KV append ------------------------------------------------------------------------ */
/* Replaces the advanced-index cache writes of flash_attn_with_kvcache
 * (flash_attn.py:480-485); graph-capturable (no host sync). */
int mykfa_kv_append(const mykfa_kv_append_params* p, mykfa_stream_t stream);

/* ---- attention-block prologue / epilogue -------------------------------------------- */
size_t mykfa_sizeof_qk_prologue_params(void);
size_t mykfa_sizeof_qk_prologue_bwd_params(void);
size_t mykfa_sizeof_gate_params(void);
int mykfa_validate_qk_prologue(const mykfa_qk_prologue_params* p);
int mykfa_validate_qk_prologue_bwd(const mykfa_qk_prologue_bwd_params* p);
int mykfa_validate_gate(const mykfa_gate_params* p, int backward);
/* q/k RMSNorm + RoPE (replaces mixers.py:85-89 with layers.py:22-25, :93-98). */
int mykfa_qk_prologue_fwd(const mykfa_qk_prologue_params* p, mykfa_stream_t stream);
/* fp32 workspace the backward needs for its weight-gradient partials (0 without norm). */
size_t mykfa_qk_prologue_bwd_workspace_size(int32_t batch, int32_t seqlen, int32_t num_heads,
                                            int32_t num_kv_heads, int32_t head_dim);
/* Gradients of the prologue (autograd of mixers.py:85-89), plus the optional dv copy. */
int mykfa_qk_prologue_bwd(const mykfa_qk_prologue_bwd_params* p, void* workspace, size_t workspace_bytes,
                          mykfa_stream_t stream);
/* y = x * sigmoid(gate) (replaces mixers.py:116-117). */
int mykfa_gate_fwd(const mykfa_gate_params* p, mykfa_stream_t stream);
/* dx, dgate from dy (autograd of mixers.py:116-117). */
int mykfa_gate_bwd(const mykfa_gate_params* p, mykfa_stream_t stream);

/* ---- fused linear + cross-entropy: the row kernel ----------------------------------- */
size_t mykfa_sizeof_ce_params(void);
int mykfa_validate_ce(const mykfa_ce_params* p);
/* lse, ce and the in-place logits gradient of each row (replaces _ce_kernel,
 * ops/fused_ce.py:20-67; launched per token chunk by _FusedLinearCE.forward, :78-89). */
int mykfa_ce_rows(const mykfa_ce_params* p, mykfa_stream_t stream);

/* ---- Muon: batched SYRK ------------------------------------------------------------ */
size_t mykfa_sizeof_syrk_params(void);
int mykfa_validate_syrk(const mykfa_syrk_params* p);
/* out = alpha x x^T + beta bias over lower-triangular tiles (replaces _batched_syrk_kernel,
 * ops/muon.py:28-104, and its launcher batched_syrk, :107-143). */
int mykfa_syrk(const mykfa_syrk_params* p, mykfa_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MYKFA_H */
