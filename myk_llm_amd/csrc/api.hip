// C ABI of libmykfa: argument validation (host only, usable without a GPU), error
// reporting, and dispatch to the kernel launchers. Nothing here allocates device memory or
// synchronizes; launches go to the caller's stream.
#include <stdarg.h>
#include <stdio.h>

#include <string>

#include "kernels.h"

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

int ok() {
    g_error.clear();
    return MYKFA_OK;
}

int launched(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(MYKFA_ERR_LAUNCH, "%s: HIP launch failed: %s", what, hipGetErrorString(e));
    return ok();
}

bool head_dim_supported(int d) { return d == 16 || d == 32 || d == 64 || d == 128 || d == 256; }

// Kernels use 16-byte vector accesses along head_dim: base pointers must be 16-byte aligned
// and every stride a multiple of 8 elements.
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
bool stride_ok(int64_t s) { return s >= 0 && (s & 7) == 0; }

// The kernels address the rows of one (sequence, head) through a buffer descriptor with a
// 32-bit byte range: rows * token stride must stay within 2 GiB.
int check_tensor(const void* ptr, int64_t bs, int64_t ts, int64_t hs, const char* name, bool needed,
                 int64_t rows, int head_dim) {
    if (!needed) return MYKFA_OK;
    if (ptr == nullptr) return fail(MYKFA_ERR_INVALID, "%s is NULL", name);
    if (!aligned16(ptr)) return fail(MYKFA_ERR_INVALID, "%s must be 16-byte aligned", name);
    if (!stride_ok(bs) || !stride_ok(ts) || !stride_ok(hs))
        return fail(MYKFA_ERR_INVALID,
                    "%s strides (%lld, %lld, %lld) must be non-negative multiples of 8 elements", name,
                    (long long)bs, (long long)ts, (long long)hs);
    if (ts > (1LL << 24)) return fail(MYKFA_ERR_UNSUPPORTED, "%s token stride %lld exceeds 2^24", name, (long long)ts);
    if (rows > 0 && ((rows - 1) * ts + head_dim) * 2 > 0x7fffffffLL)
        return fail(MYKFA_ERR_UNSUPPORTED, "%s: %lld rows at token stride %lld span more than 2 GiB", name,
                    (long long)rows, (long long)ts);
    return MYKFA_OK;
}

// flash_attn.py:336-346 (_check) and the layout rules of _forward (:358-363).
int check_fwd(const mykfa_fwd_params* p) {
    if (p == nullptr) return fail(MYKFA_ERR_INVALID, "params is NULL");
    if (p->dtype != MYKFA_BF16 && p->dtype != MYKFA_FP16)
        return fail(MYKFA_ERR_UNSUPPORTED, "flash attention needs bf16/fp16 q, k, v; got dtype code %d", p->dtype);
    if (!head_dim_supported(p->head_dim))
        return fail(MYKFA_ERR_UNSUPPORTED, "head_dim must be one of [16, 32, 64, 128, 256]; got %d", p->head_dim);
    if (p->num_heads <= 0 || p->num_kv_heads <= 0 || p->num_heads % p->num_kv_heads != 0)
        return fail(MYKFA_ERR_INVALID, "query heads (%d) must be a multiple of key/value heads (%d)", p->num_heads,
                    p->num_kv_heads);
    if (p->num_heads > 65535 * 4)
        return fail(MYKFA_ERR_UNSUPPORTED, "num_heads %d exceeds the grid limit", p->num_heads);
    if (p->batch < 0 || p->max_seqlen_q < 0 || p->max_seqlen_k < 0)
        return fail(MYKFA_ERR_INVALID, "negative batch (%d) or sequence length (%d, %d)", p->batch, p->max_seqlen_q,
                    p->max_seqlen_k);
    if (p->batch > 65535) return fail(MYKFA_ERR_UNSUPPORTED, "batch %d exceeds the grid limit 65535", p->batch);
    if (p->window_left < 0 || p->window_right < 0 || p->window_left > MYKFA_UNBOUNDED ||
        p->window_right > MYKFA_UNBOUNDED)
        return fail(MYKFA_ERR_INVALID, "window sides must lie in [0, 2^30]; got (%d, %d)", p->window_left,
                    p->window_right);
    if (!(p->softmax_scale == p->softmax_scale)) return fail(MYKFA_ERR_INVALID, "softmax_scale is NaN");
    const bool varlen_q = p->cu_seqlens_q != nullptr, varlen_k = p->cu_seqlens_k != nullptr;
    if (varlen_q != varlen_k)
        return fail(MYKFA_ERR_INVALID, "cu_seqlens_q and cu_seqlens_k must both be given or both be NULL");
    if (varlen_q && p->seqused_k != nullptr)
        return fail(MYKFA_ERR_INVALID, "seqused_k applies to the dense layout only");
    if (varlen_q && (p->q_batch_stride != 0 || p->k_batch_stride != 0 || p->v_batch_stride != 0 ||
                     p->o_batch_stride != 0))
        return fail(MYKFA_ERR_INVALID, "packed (varlen) tensors must have batch stride 0");
    const bool work = p->batch > 0 && p->max_seqlen_q > 0;
    int rc;
    if ((rc = check_tensor(p->q, p->q_batch_stride, p->q_token_stride, p->q_head_stride, "q", work, p->max_seqlen_q, p->head_dim))) return rc;
    if ((rc = check_tensor(p->o, p->o_batch_stride, p->o_token_stride, p->o_head_stride, "o", work, p->max_seqlen_q, p->head_dim))) return rc;
    const bool keys = work && p->max_seqlen_k > 0;
    if ((rc = check_tensor(p->k, p->k_batch_stride, p->k_token_stride, p->k_head_stride, "k", keys, p->max_seqlen_k, p->head_dim))) return rc;
    if ((rc = check_tensor(p->v, p->v_batch_stride, p->v_token_stride, p->v_head_stride, "v", keys, p->max_seqlen_k, p->head_dim))) return rc;
    if (work && p->lse == nullptr) return fail(MYKFA_ERR_INVALID, "lse is NULL");
    if (work && p->lse_head_stride < (varlen_q ? 0 : (int64_t)p->batch * p->max_seqlen_q))
        return fail(MYKFA_ERR_INVALID, "lse_head_stride %lld is smaller than the number of rows",
                    (long long)p->lse_head_stride);
    return ok();
}

int check_bwd(const mykfa_bwd_params* p) {
    if (p == nullptr) return fail(MYKFA_ERR_INVALID, "params is NULL");
    int rc = check_fwd(&p->fwd);
    if (rc) return rc;
    if (p->fwd.seqused_k != nullptr) return fail(MYKFA_ERR_INVALID, "the backward pass takes no seqused_k");
    const bool work = p->fwd.batch > 0 && p->fwd.max_seqlen_q > 0;
    const bool keys = p->fwd.batch > 0 && p->fwd.max_seqlen_k > 0;
    if ((rc = check_tensor(p->dout, p->do_batch_stride, p->do_token_stride, p->do_head_stride, "dout", work, p->fwd.max_seqlen_q, p->fwd.head_dim))) return rc;
    if ((rc = check_tensor(p->dq, p->dq_batch_stride, p->dq_token_stride, p->dq_head_stride, "dq", work, p->fwd.max_seqlen_q, p->fwd.head_dim))) return rc;
    if ((rc = check_tensor(p->dk, p->dk_batch_stride, p->dk_token_stride, p->dk_head_stride, "dk", keys, p->fwd.max_seqlen_k, p->fwd.head_dim))) return rc;
    if ((rc = check_tensor(p->dv, p->dv_batch_stride, p->dv_token_stride, p->dv_head_stride, "dv", keys, p->fwd.max_seqlen_k, p->fwd.head_dim))) return rc;
    if (work && p->delta == nullptr) return fail(MYKFA_ERR_INVALID, "delta is NULL");
    if (p->fwd.cu_seqlens_q != nullptr &&
        (p->do_batch_stride != 0 || p->dq_batch_stride != 0 || p->dk_batch_stride != 0 || p->dv_batch_stride != 0))
        return fail(MYKFA_ERR_INVALID, "packed (varlen) gradients must have batch stride 0");
    return ok();
}

int check_decode(const mykfa_decode_params* p) {
    if (p == nullptr) return fail(MYKFA_ERR_INVALID, "params is NULL");
    int rc = check_fwd(&p->fwd);
    if (rc) return rc;
    if (p->fwd.cu_seqlens_q != nullptr) return fail(MYKFA_ERR_INVALID, "decode takes the dense layout only");
    if (p->num_splits < 0 || p->num_splits > 1024)
        return fail(MYKFA_ERR_INVALID, "num_splits must lie in [0, 1024]; got %d", p->num_splits);
    if (p->seqlen_new < 0) return fail(MYKFA_ERR_INVALID, "seqlen_new must be >= 0; got %d", p->seqlen_new);
    if (p->seqlen_new > 0 && p->fwd.seqused_k == nullptr)
        return fail(MYKFA_ERR_INVALID, "seqlen_new > 0 needs seqused_k (the cached lengths)");
    if ((p->k_new == nullptr) != (p->v_new == nullptr))
        return fail(MYKFA_ERR_INVALID, "k_new and v_new must both be given or both be NULL");
    const bool append = p->k_new != nullptr && p->seqlen_new > 0 && p->fwd.batch > 0;
    if ((rc = check_tensor(p->k_new, p->kn_batch_stride, p->kn_token_stride, p->kn_head_stride, "k_new", append,
                           p->seqlen_new, p->fwd.head_dim)))
        return rc;
    if ((rc = check_tensor(p->v_new, p->vn_batch_stride, p->vn_token_stride, p->vn_head_stride, "v_new", append,
                           p->seqlen_new, p->fwd.head_dim)))
        return rc;
    if (append && (p->fwd.k == nullptr || p->fwd.v == nullptr))
        return fail(MYKFA_ERR_INVALID, "appending new keys needs the caches k and v");
    return ok();
}

int check_append(const mykfa_kv_append_params* p) {
    if (p == nullptr) return fail(MYKFA_ERR_INVALID, "params is NULL");
    if (p->dtype != MYKFA_BF16 && p->dtype != MYKFA_FP16)
        return fail(MYKFA_ERR_UNSUPPORTED, "kv append needs bf16/fp16 caches; got dtype code %d", p->dtype);
    if (!head_dim_supported(p->head_dim))
        return fail(MYKFA_ERR_UNSUPPORTED, "head_dim must be one of [16, 32, 64, 128, 256]; got %d", p->head_dim);
    if (p->batch < 0 || p->seqlen_new < 0 || p->capacity < 0 || p->num_kv_heads <= 0)
        return fail(MYKFA_ERR_INVALID, "invalid kv append shape");
    if (p->batch > 65535) return fail(MYKFA_ERR_UNSUPPORTED, "batch %d exceeds the grid limit 65535", p->batch);
    const bool work = p->batch > 0 && p->seqlen_new > 0;
    if (work && p->cache_seqlens == nullptr) return fail(MYKFA_ERR_INVALID, "cache_seqlens is NULL");
    int rc;
    if ((rc = check_tensor(p->k_cache, p->kc_batch_stride, p->kc_token_stride, p->kc_head_stride, "k_cache", work, p->capacity, p->head_dim))) return rc;
    if ((rc = check_tensor(p->v_cache, p->vc_batch_stride, p->vc_token_stride, p->vc_head_stride, "v_cache", work, p->capacity, p->head_dim))) return rc;
    if ((rc = check_tensor(p->k_new, p->kn_batch_stride, p->kn_token_stride, p->kn_head_stride, "k", work, p->seqlen_new, p->head_dim))) return rc;
    if ((rc = check_tensor(p->v_new, p->vn_batch_stride, p->vn_token_stride, p->vn_head_stride, "v", work, p->seqlen_new, p->head_dim))) return rc;
    return ok();
}

// A (batch, token, head) view read or written 16 bytes at a time by the elementwise kernels
// (64-bit addressing: no span limit).
int check_view(const void* ptr, int64_t bs, int64_t ts, int64_t hs, const char* name) {
    if (ptr == nullptr) return fail(MYKFA_ERR_INVALID, "%s is NULL", name);
    if (!aligned16(ptr)) return fail(MYKFA_ERR_INVALID, "%s must be 16-byte aligned", name);
    if (!stride_ok(bs) || !stride_ok(ts) || !stride_ok(hs))
        return fail(MYKFA_ERR_INVALID, "%s strides (%lld, %lld, %lld) must be non-negative multiples of 8 elements",
                    name, (long long)bs, (long long)ts, (long long)hs);
    return MYKFA_OK;
}

// mixers.py:85-89 with RMSNorm (layers.py:15-25) and RotaryEmbedding (layers.py:73-101).
// `outputs`: whether q_out/k_out are written (the backward ignores them).
int check_prologue(const mykfa_qk_prologue_params* p, bool outputs = true) {
    if (p == nullptr) return fail(MYKFA_ERR_INVALID, "params is NULL");
    if (p->dtype != MYKFA_BF16 && p->dtype != MYKFA_FP16)
        return fail(MYKFA_ERR_UNSUPPORTED, "the q/k prologue needs bf16/fp16 q, k; got dtype code %d", p->dtype);
    if (!head_dim_supported(p->head_dim))
        return fail(MYKFA_ERR_UNSUPPORTED, "head_dim must be one of [16, 32, 64, 128, 256]; got %d", p->head_dim);
    if (p->batch < 0 || p->seqlen < 0 || p->num_heads < 0 || p->num_kv_heads < 0)
        return fail(MYKFA_ERR_INVALID, "negative shape (batch %d, seqlen %d, heads %d, kv heads %d)", p->batch,
                    p->seqlen, p->num_heads, p->num_kv_heads);
    if ((p->q_weight == nullptr) != (p->k_weight == nullptr))
        return fail(MYKFA_ERR_INVALID, "q_weight and k_weight must both be given or both be NULL");
    if ((p->cos == nullptr) != (p->sin == nullptr))
        return fail(MYKFA_ERR_INVALID, "cos and sin must both be given or both be NULL");
    const bool work = p->batch > 0 && p->seqlen > 0 && p->num_heads + p->num_kv_heads > 0;
    if (!work) return MYKFA_OK;
    int rc;
    if (p->num_heads > 0) {
        if ((rc = check_view(p->q_in, p->qi_batch_stride, p->qi_token_stride, p->qi_head_stride, "q_in"))) return rc;
        if (outputs && (rc = check_view(p->q_out, p->qo_batch_stride, p->qo_token_stride, p->qo_head_stride, "q_out"))) return rc;
    }
    if (p->num_kv_heads > 0) {
        if ((rc = check_view(p->k_in, p->ki_batch_stride, p->ki_token_stride, p->ki_head_stride, "k_in"))) return rc;
        if (outputs && (rc = check_view(p->k_out, p->ko_batch_stride, p->ko_token_stride, p->ko_head_stride, "k_out"))) return rc;
    }
    if (p->q_weight != nullptr) {
        if (!aligned16(p->q_weight) || !aligned16(p->k_weight))
            return fail(MYKFA_ERR_INVALID, "q_weight and k_weight must be 16-byte aligned");
        if (!(p->eps >= 0.0f) || p->eps > 1e30f) return fail(MYKFA_ERR_INVALID, "eps must be finite and >= 0");
    }
    if (p->cos != nullptr) {
        if (p->position_ids == nullptr) return fail(MYKFA_ERR_INVALID, "position_ids is NULL");
        if ((reinterpret_cast<uintptr_t>(p->position_ids) & 7) != 0)
            return fail(MYKFA_ERR_INVALID, "position_ids must be 8-byte aligned int64");
        if (p->pos_batch_stride < 0 || p->pos_token_stride < 0)
            return fail(MYKFA_ERR_INVALID, "position_ids strides must be non-negative");
        if (!aligned16(p->cos) || !aligned16(p->sin))
            return fail(MYKFA_ERR_INVALID, "cos and sin tables must be 16-byte aligned");
        if (p->table_rows <= 0) return fail(MYKFA_ERR_INVALID, "table_rows must be positive; got %d", p->table_rows);
        if (p->table_stride < p->head_dim || (p->table_stride & 3) != 0)
            return fail(MYKFA_ERR_INVALID, "table_stride %lld must be >= head_dim and a multiple of 4",
                        (long long)p->table_stride);
    }
    return MYKFA_OK;
}

int check_prologue_bwd(const mykfa_qk_prologue_bwd_params* p) {
    if (p == nullptr) return fail(MYKFA_ERR_INVALID, "params is NULL");
    int rc = check_prologue(&p->fwd, false);
    if (rc) return rc;
    const mykfa_qk_prologue_params& f = p->fwd;
    if ((p->dv_src == nullptr) != (p->dv_dst == nullptr))
        return fail(MYKFA_ERR_INVALID, "dv_src and dv_dst must both be given or both be NULL");
    if (f.q_weight != nullptr && (p->dq_weight == nullptr || p->dk_weight == nullptr))
        return fail(MYKFA_ERR_INVALID, "dq_weight and dk_weight are required when the forward had weights");
    const bool work = f.batch > 0 && f.seqlen > 0;
    if (!work) return MYKFA_OK;
    if (f.num_heads > 0) {
        if ((rc = check_view(p->dq_out, p->dqo_batch_stride, p->dqo_token_stride, p->dqo_head_stride, "dq_out"))) return rc;
        if ((rc = check_view(p->dq_in, p->dqi_batch_stride, p->dqi_token_stride, p->dqi_head_stride, "dq_in"))) return rc;
    }
    if (f.num_kv_heads > 0) {
        if ((rc = check_view(p->dk_out, p->dko_batch_stride, p->dko_token_stride, p->dko_head_stride, "dk_out"))) return rc;
        if ((rc = check_view(p->dk_in, p->dki_batch_stride, p->dki_token_stride, p->dki_head_stride, "dk_in"))) return rc;
        if (p->dv_src != nullptr) {
            if ((rc = check_view(p->dv_src, p->dvs_batch_stride, p->dvs_token_stride, p->dvs_head_stride, "dv_src"))) return rc;
            if ((rc = check_view(p->dv_dst, p->dvd_batch_stride, p->dvd_token_stride, p->dvd_head_stride, "dv_dst"))) return rc;
        }
    }
    return MYKFA_OK;
}

// mixers.py:116-117.
int check_gate(const mykfa_gate_params* p, bool backward) {
    if (p == nullptr) return fail(MYKFA_ERR_INVALID, "params is NULL");
    if (p->dtype != MYKFA_BF16 && p->dtype != MYKFA_FP16)
        return fail(MYKFA_ERR_UNSUPPORTED, "the output gate needs bf16/fp16 tensors; got dtype code %d", p->dtype);
    if (p->rows < 0 || p->width <= 0 || (p->width & 7) != 0)
        return fail(MYKFA_ERR_INVALID, "rows (%lld) must be >= 0 and width (%d) a positive multiple of 8",
                    (long long)p->rows, p->width);
    if (p->rows == 0) return MYKFA_OK;
    int rc;
    if ((rc = check_view(p->x, 0, p->x_row_stride, 0, "x"))) return rc;
    if ((rc = check_view(p->gate, 0, p->gate_row_stride, 0, "gate"))) return rc;
    if (!backward) return check_view(p->y, 0, p->y_row_stride, 0, "y");
    if ((rc = check_view(p->dy, 0, p->dy_row_stride, 0, "dy"))) return rc;
    if ((rc = check_view(p->dx, 0, p->dx_row_stride, 0, "dx"))) return rc;
    return check_view(p->dgate, 0, p->dgate_row_stride, 0, "dgate");
}

// ops/fused_ce.py:20-33 (the row kernel's arguments).
int check_ce(const mykfa_ce_params* p) {
    if (p == nullptr) return fail(MYKFA_ERR_INVALID, "params is NULL");
    if (p->dtype != MYKFA_BF16 && p->dtype != MYKFA_FP16)
        return fail(MYKFA_ERR_UNSUPPORTED, "cross entropy needs bf16/fp16 logits; got dtype code %d", p->dtype);
    if (p->rows < 0 || p->rows > 0x7fffffffLL)
        return fail(MYKFA_ERR_INVALID, "rows must lie in [0, 2^31); got %lld", (long long)p->rows);
    if (p->vocab <= 0) return fail(MYKFA_ERR_INVALID, "vocab must be positive; got %d", p->vocab);
    if (p->rows == 0) return MYKFA_OK;
    if (p->row_stride < p->vocab)
        return fail(MYKFA_ERR_INVALID, "row_stride %lld is smaller than vocab %d", (long long)p->row_stride, p->vocab);
    if (p->logits == nullptr || p->targets == nullptr || p->ce == nullptr || p->lse == nullptr)
        return fail(MYKFA_ERR_INVALID, "logits, targets, ce and lse must be non-NULL");
    if ((reinterpret_cast<uintptr_t>(p->logits) & 1) != 0 || (reinterpret_cast<uintptr_t>(p->targets) & 7) != 0 ||
        (reinterpret_cast<uintptr_t>(p->ce) & 3) != 0 || (reinterpret_cast<uintptr_t>(p->lse) & 3) != 0)
        return fail(MYKFA_ERR_INVALID, "misaligned logits / targets / ce / lse");
    if (!(p->scale == p->scale) || !(p->z_coef == p->z_coef)) return fail(MYKFA_ERR_INVALID, "scale or z_coef is NaN");
    return MYKFA_OK;
}

// ops/muon.py:107-143 (batched_syrk's arguments) with this kernel's layout rules.
int check_syrk(const mykfa_syrk_params* p) {
    if (p == nullptr) return fail(MYKFA_ERR_INVALID, "params is NULL");
    if (p->dtype != MYKFA_BF16) return fail(MYKFA_ERR_UNSUPPORTED, "batched SYRK needs bf16 x; got dtype code %d", p->dtype);
    if (p->batch < 0 || p->m < 0 || p->k < 0)
        return fail(MYKFA_ERR_INVALID, "negative shape (batch %d, m %d, k %d)", p->batch, p->m, p->k);
    {
        const long long t = ((long long)p->m + 127) / 128;
        if ((long long)p->batch * (t * (t + 1) / 2) > 0x7ffffff0LL)
            return fail(MYKFA_ERR_UNSUPPORTED, "batch %d x %lld output tiles exceed the grid limit", p->batch, t * (t + 1) / 2);
    }
    if (p->k % 64 != 0) return fail(MYKFA_ERR_UNSUPPORTED, "k (%d) must be a multiple of 64: pad x with zero columns", p->k);
    if (!(p->alpha == p->alpha) || !(p->beta == p->beta)) return fail(MYKFA_ERR_INVALID, "alpha or beta is NaN");
    if (p->batch == 0 || p->m == 0) return MYKFA_OK;
    if (p->out == nullptr || (reinterpret_cast<uintptr_t>(p->out) & 7) != 0)
        return fail(MYKFA_ERR_INVALID, "out must be non-NULL and 8-byte aligned");
    if (p->out_row_stride < p->m || (p->out_row_stride & 3) != 0 || p->out_batch_stride < 0)
        return fail(MYKFA_ERR_INVALID, "out row stride %lld must be >= m and a multiple of 4", (long long)p->out_row_stride);
    if (p->bias != nullptr && ((reinterpret_cast<uintptr_t>(p->bias) & 1) != 0 || p->bias_row_stride < 0 ||
                               p->bias_batch_stride < 0))
        return fail(MYKFA_ERR_INVALID, "bias must be 2-byte aligned with non-negative strides");
    if (p->k == 0) return MYKFA_OK;
    if (p->x == nullptr || !aligned16(p->x)) return fail(MYKFA_ERR_INVALID, "x must be non-NULL and 16-byte aligned");
    if (p->x_row_stride < p->k || (p->x_row_stride & 7) != 0 || p->x_batch_stride < 0)
        return fail(MYKFA_ERR_INVALID, "x row stride %lld must be >= k and a multiple of 8", (long long)p->x_row_stride);
    if ((127 * p->x_row_stride + p->k) * 2 > 0x7fffffffLL)
        return fail(MYKFA_ERR_UNSUPPORTED, "128 rows of x at row stride %lld span more than 2 GiB", (long long)p->x_row_stride);
    return MYKFA_OK;
}

hipStream_t as_stream(mykfa_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

int choose_splits(const mykfa_decode_params* p) {
    return p->num_splits > 0 ? p->num_splits
                             : mykfa::decode_default_splits(p->fwd.batch, p->fwd.num_heads, p->fwd.num_kv_heads,
                                                            p->fwd.max_seqlen_q, p->fwd.max_seqlen_k);
}

}  // namespace

extern "C" {

int mykfa_abi_version(void) { return MYKFA_ABI_VERSION; }
const char* mykfa_version(void) { return "mykfa 0.1.0 (gfx950)"; }
const char* mykfa_last_error(void) { return g_error.c_str(); }
size_t mykfa_sizeof_fwd_params(void) { return sizeof(mykfa_fwd_params); }
size_t mykfa_sizeof_bwd_params(void) { return sizeof(mykfa_bwd_params); }
size_t mykfa_sizeof_decode_params(void) { return sizeof(mykfa_decode_params); }
size_t mykfa_sizeof_kv_append_params(void) { return sizeof(mykfa_kv_append_params); }

int mykfa_validate_fwd(const mykfa_fwd_params* p) { return check_fwd(p); }
int mykfa_validate_bwd(const mykfa_bwd_params* p) { return check_bwd(p); }
int mykfa_validate_decode(const mykfa_decode_params* p) { return check_decode(p); }
int mykfa_validate_kv_append(const mykfa_kv_append_params* p) { return check_append(p); }

int mykfa_fwd(const mykfa_fwd_params* p, mykfa_stream_t stream) {
    int rc = check_fwd(p);
    if (rc) return rc;
    if (p->batch == 0 || p->max_seqlen_q == 0) return ok();
    return launched(mykfa::launch_fwd(*p, as_stream(stream)), "mykfa_fwd");
}

int mykfa_bwd_preprocess(const mykfa_bwd_params* p, mykfa_stream_t stream) {
    int rc = check_bwd(p);
    if (rc) return rc;
    if (p->fwd.batch == 0 || p->fwd.max_seqlen_q == 0) return ok();
    return launched(mykfa::launch_bwd_preprocess(*p, as_stream(stream)), "mykfa_bwd_preprocess");
}

int mykfa_bwd_dkdv(const mykfa_bwd_params* p, mykfa_stream_t stream) {
    int rc = check_bwd(p);
    if (rc) return rc;
    if (p->fwd.batch == 0 || p->fwd.max_seqlen_k == 0) return ok();
    return launched(mykfa::launch_bwd_dkdv(*p, as_stream(stream)), "mykfa_bwd_dkdv");
}

int mykfa_bwd_dq(const mykfa_bwd_params* p, mykfa_stream_t stream) {
    int rc = check_bwd(p);
    if (rc) return rc;
    if (p->fwd.batch == 0 || p->fwd.max_seqlen_q == 0) return ok();
    return launched(mykfa::launch_bwd_dq(*p, as_stream(stream)), "mykfa_bwd_dq");
}

int mykfa_bwd(const mykfa_bwd_params* p, mykfa_stream_t stream) {
    // dQ first: it computes delta (the preprocess) itself and writes it for dK/dV.
    int rc = mykfa_bwd_dq(p, stream);
    if (rc) return rc;
    return mykfa_bwd_dkdv(p, stream);
}

size_t mykfa_bwd_workspace_per_kv_head(const mykfa_bwd_params* p) {
    if (check_bwd(p)) return 0;
    return mykfa::bwd_ds_bytes_per_kv_head(*p);
}

int mykfa_bwd_ws(const mykfa_bwd_params* p, void* workspace, size_t workspace_bytes, mykfa_stream_t stream) {
    int rc = check_bwd(p);
    if (rc) return rc;
    const size_t per = mykfa::bwd_ds_bytes_per_kv_head(*p);
    if (per == 0 || workspace_bytes < per) return mykfa_bwd(p, stream);
    if (workspace == nullptr) return fail(MYKFA_ERR_INVALID, "workspace is NULL");
    // dS blocks are written and read as 16-byte chunks and the block-queue counters take
    // device-scope atomics: the buffer must be 16-byte aligned.
    if (!aligned16(workspace)) return fail(MYKFA_ERR_INVALID, "mykfa_bwd_ws: workspace must be 16-byte aligned");
    const size_t heads = workspace_bytes / per;
    const int per_pass = heads < (size_t)p->fwd.num_kv_heads ? (int)heads : p->fwd.num_kv_heads;
    return launched(mykfa::launch_bwd_ds(*p, workspace, per_pass, as_stream(stream)), "mykfa_bwd_ws");
}

namespace {
int bwd_ds_half(const mykfa_bwd_params* p, void* workspace, size_t workspace_bytes, mykfa_stream_t stream,
                bool dq, const char* what) {
    int rc = check_bwd(p);
    if (rc) return rc;
    const size_t per = mykfa::bwd_ds_bytes_per_kv_head(*p);
    if (per == 0) return fail(MYKFA_ERR_UNSUPPORTED, "%s: no stored-dS path for head_dim %d", what, p->fwd.head_dim);
    const size_t need = per * (size_t)p->fwd.num_kv_heads;
    if (workspace_bytes < need)
        return fail(MYKFA_ERR_WORKSPACE, "%s: workspace of %zu bytes, %zu needed (every KV head's dS)", what,
                    workspace_bytes, need);
    if (workspace == nullptr) return fail(MYKFA_ERR_INVALID, "workspace is NULL");
    if (!aligned16(workspace)) return fail(MYKFA_ERR_INVALID, "%s: workspace must be 16-byte aligned", what);
    return launched(mykfa::launch_bwd_ds_half(*p, workspace, dq, as_stream(stream)), what);
}
}  // namespace

int mykfa_bwd_dkdv_ws(const mykfa_bwd_params* p, void* workspace, size_t workspace_bytes, mykfa_stream_t stream) {
    return bwd_ds_half(p, workspace, workspace_bytes, stream, false, "mykfa_bwd_dkdv_ws");
}

int mykfa_bwd_dq_ws(const mykfa_bwd_params* p, void* workspace, size_t workspace_bytes, mykfa_stream_t stream) {
    return bwd_ds_half(p, workspace, workspace_bytes, stream, true, "mykfa_bwd_dq_ws");
}

int mykfa_decode_num_splits(int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t seqlen_q,
                            int32_t capacity) {
    return mykfa::decode_default_splits(batch, num_heads, num_kv_heads, seqlen_q, capacity);
}

size_t mykfa_decode_workspace_size(int32_t batch, int32_t num_heads, int32_t seqlen_q, int32_t head_dim,
                                   int32_t num_splits) {
    if (batch < 0 || num_heads < 0 || seqlen_q < 0 || head_dim < 0 || num_splits < 0) return 0;
    return mykfa::decode_workspace_bytes(batch, num_heads, seqlen_q, head_dim, num_splits);
}

int mykfa_decode_splitk(const mykfa_decode_params* p, void* workspace, size_t workspace_bytes,
                        mykfa_stream_t stream) {
    int rc = check_decode(p);
    if (rc) return rc;
    if (p->fwd.batch == 0 || p->fwd.max_seqlen_q == 0) return ok();
    const int splits = choose_splits(p);
    const size_t need = mykfa::decode_workspace_bytes(p->fwd.batch, p->fwd.num_heads, p->fwd.max_seqlen_q,
                                                      p->fwd.head_dim, splits);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
        return fail(MYKFA_ERR_WORKSPACE, "decode workspace needs %zu bytes; got %zu", need, workspace_bytes);
    if (!aligned16(workspace)) return fail(MYKFA_ERR_INVALID, "workspace must be 16-byte aligned");
    return launched(mykfa::launch_decode_splitk(*p, splits, workspace, as_stream(stream)), "mykfa_decode_splitk");
}

int mykfa_decode_merge(const mykfa_decode_params* p, const void* workspace, size_t workspace_bytes,
                       mykfa_stream_t stream) {
    int rc = check_decode(p);
    if (rc) return rc;
    if (p->fwd.batch == 0 || p->fwd.max_seqlen_q == 0) return ok();
    const int splits = choose_splits(p);
    const size_t need = mykfa::decode_workspace_bytes(p->fwd.batch, p->fwd.num_heads, p->fwd.max_seqlen_q,
                                                      p->fwd.head_dim, splits);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
        return fail(MYKFA_ERR_WORKSPACE, "decode workspace needs %zu bytes; got %zu", need, workspace_bytes);
    return launched(mykfa::launch_decode_merge(*p, splits, workspace, as_stream(stream)), "mykfa_decode_merge");
}

int mykfa_decode(const mykfa_decode_params* p, void* workspace, size_t workspace_bytes, mykfa_stream_t stream) {
    int rc = mykfa_decode_splitk(p, workspace, workspace_bytes, stream);
    if (rc) return rc;
    if (choose_splits(p) == 1) return ok();  // a single split writes o and lse directly
    return mykfa_decode_merge(p, workspace, workspace_bytes, stream);
}

int mykfa_decode_noalloc(const mykfa_decode_params* p, mykfa_stream_t stream) {
    int rc = check_decode(p);
    if (rc) return rc;
    if (p->fwd.batch == 0 || p->fwd.max_seqlen_q == 0) return ok();
    const size_t cap = MYKFA_DECODE_SCRATCH_BYTES;
    const size_t per_split = mykfa::decode_workspace_bytes(p->fwd.batch, p->fwd.num_heads, p->fwd.max_seqlen_q,
                                                           p->fwd.head_dim, 2) / 2;
    int splits = choose_splits(p);
    if (p->num_splits > 0) {
        const size_t need = mykfa::decode_workspace_bytes(p->fwd.batch, p->fwd.num_heads, p->fwd.max_seqlen_q,
                                                          p->fwd.head_dim, splits);
        if (need > cap)
            return fail(MYKFA_ERR_WORKSPACE,
                        "mykfa_decode_noalloc: %d splits need %zu bytes of scratch, beyond its fixed %zu bytes "
                        "(use fewer splits, num_splits = 0, or mykfa_decode with a workspace)",
                        splits, need, cap);
    } else if (per_split > 0 && (size_t)splits * per_split > cap) {
        // The library's own choice is cut to what the scratch holds (off multiples of the 8 XCDs).
        splits = (int)(cap / per_split);
        if (splits > 1 && splits % 8 == 0) --splits;
        if (splits < 1) splits = 1;
    }
    void* ws = nullptr;
    if (splits > 1) {
        const hipError_t e = mykfa::decode_scratch(as_stream(stream), &ws);
        if (e != hipSuccess)
            return fail(MYKFA_ERR_LAUNCH, "mykfa_decode_noalloc: scratch address: %s", hipGetErrorString(e));
    }
    mykfa_decode_params q = *p;
    q.num_splits = splits;
    rc = launched(mykfa::launch_decode_splitk(q, splits, ws, as_stream(stream)), "mykfa_decode_noalloc");
    if (rc || splits == 1) return rc;
    return launched(mykfa::launch_decode_merge(q, splits, ws, as_stream(stream)), "mykfa_decode_noalloc");
}

int mykfa_kv_append(const mykfa_kv_append_params* p, mykfa_stream_t stream) {
    int rc = check_append(p);
    if (rc) return rc;
    if (p->batch == 0 || p->seqlen_new == 0) return ok();
    return launched(mykfa::launch_kv_append(*p, as_stream(stream)), "mykfa_kv_append");
}

size_t mykfa_sizeof_qk_prologue_params(void) { return sizeof(mykfa_qk_prologue_params); }
size_t mykfa_sizeof_qk_prologue_bwd_params(void) { return sizeof(mykfa_qk_prologue_bwd_params); }
size_t mykfa_sizeof_gate_params(void) { return sizeof(mykfa_gate_params); }

int mykfa_validate_qk_prologue(const mykfa_qk_prologue_params* p) {
    int rc = check_prologue(p);
    return rc ? rc : ok();
}
int mykfa_validate_qk_prologue_bwd(const mykfa_qk_prologue_bwd_params* p) {
    int rc = check_prologue_bwd(p);
    return rc ? rc : ok();
}
int mykfa_validate_gate(const mykfa_gate_params* p, int backward) {
    int rc = check_gate(p, backward != 0);
    return rc ? rc : ok();
}

int mykfa_qk_prologue_fwd(const mykfa_qk_prologue_params* p, mykfa_stream_t stream) {
    int rc = check_prologue(p);
    if (rc) return rc;
    if ((long long)p->batch * p->seqlen * (p->num_heads + p->num_kv_heads) == 0) return ok();
    return launched(mykfa::launch_qk_prologue_fwd(*p, as_stream(stream)), "mykfa_qk_prologue_fwd");
}

size_t mykfa_qk_prologue_bwd_workspace_size(int32_t batch, int32_t seqlen, int32_t num_heads, int32_t num_kv_heads,
                                            int32_t head_dim) {
    if (batch < 0 || seqlen < 0 || num_heads < 0 || num_kv_heads < 0 || !head_dim_supported(head_dim)) return 0;
    return mykfa::qk_prologue_bwd_workspace_bytes(batch, seqlen, num_heads, num_kv_heads, head_dim);
}

int mykfa_qk_prologue_bwd(const mykfa_qk_prologue_bwd_params* p, void* workspace, size_t workspace_bytes,
                          mykfa_stream_t stream) {
    int rc = check_prologue_bwd(p);
    if (rc) return rc;
    const mykfa_qk_prologue_params& f = p->fwd;
    // With no rows and no norm there is nothing to write; with a norm the launch still writes
    // the (zero) weight gradients.
    if ((long long)f.batch * f.seqlen * (f.num_heads + f.num_kv_heads) == 0 && f.q_weight == nullptr) return ok();
    if (f.q_weight != nullptr) {
        const size_t need = (size_t)mykfa::qk_prologue_bwd_blocks(f.batch, f.seqlen, f.num_heads, f.num_kv_heads,
                                                                  f.head_dim) *
                            2 * f.head_dim * sizeof(float);
        if (workspace == nullptr || workspace_bytes < need)
            return fail(MYKFA_ERR_WORKSPACE, "prologue backward workspace needs %zu bytes; got %zu", need,
                        workspace_bytes);
        if (!aligned16(workspace)) return fail(MYKFA_ERR_INVALID, "workspace must be 16-byte aligned");
    }
    return launched(mykfa::launch_qk_prologue_bwd(*p, workspace, as_stream(stream)), "mykfa_qk_prologue_bwd");
}

int mykfa_gate_fwd(const mykfa_gate_params* p, mykfa_stream_t stream) {
    int rc = check_gate(p, false);
    if (rc) return rc;
    if (p->rows == 0) return ok();
    return launched(mykfa::launch_gate(*p, false, as_stream(stream)), "mykfa_gate_fwd");
}

int mykfa_gate_bwd(const mykfa_gate_params* p, mykfa_stream_t stream) {
    int rc = check_gate(p, true);
    if (rc) return rc;
    if (p->rows == 0) return ok();
    return launched(mykfa::launch_gate(*p, true, as_stream(stream)), "mykfa_gate_bwd");
}

size_t mykfa_sizeof_syrk_params(void) { return sizeof(mykfa_syrk_params); }

int mykfa_validate_syrk(const mykfa_syrk_params* p) {
    int rc = check_syrk(p);
    return rc ? rc : ok();
}

int mykfa_syrk(const mykfa_syrk_params* p, mykfa_stream_t stream) {
    int rc = check_syrk(p);
    if (rc) return rc;
    if (p->batch == 0 || p->m == 0) return ok();
    return launched(mykfa::launch_syrk(*p, as_stream(stream)), "mykfa_syrk");
}

size_t mykfa_sizeof_ce_params(void) { return sizeof(mykfa_ce_params); }

int mykfa_validate_ce(const mykfa_ce_params* p) {
    int rc = check_ce(p);
    return rc ? rc : ok();
}

int mykfa_ce_rows(const mykfa_ce_params* p, mykfa_stream_t stream) {
    int rc = check_ce(p);
    if (rc) return rc;
    if (p->rows == 0) return ok();
    return launched(mykfa::launch_ce_rows(*p, as_stream(stream)), "mykfa_ce_rows");
}

}  // extern "C"
