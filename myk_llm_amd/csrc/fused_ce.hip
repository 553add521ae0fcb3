// Cross-entropy rows of the fused linear + cross-entropy (replaces _ce_kernel,
// ops/fused_ce.py:20-67). One workgroup of 512 lanes per logits row:
//   lse = logsumexp(row), ce = lse - row[target] (fp32), and the row overwritten in place with
//   d loss / d logits = softmax(row) * scale * (1 + 2 z lse) - scale * onehot(target);
//   an ignored row (target == ignore_index) gets zeros, ce = lse = 0.
// ce_rows_resident_kernel: rows of up to 512 * VPT columns (65536 at VPT = 128, the
//   reference's 64K vocabulary) are held in registers, so each logit is read from HBM once and
//   written once (the reference streams the row twice: one pass for the statistics, one for the
//   gradient). 16-byte accesses: the vocabulary and the row stride are multiples of 8.
// ce_rows_stream_kernel: any other shape (larger vocabularies, unaligned rows): two passes
//   over the row, an online max/sum per lane first.
// Block reductions are fixed-order (lane shuffles, then the 8 waves in order through LDS):
// results are bitwise repeatable.
#include <math.h>

#include "common.h"
#include "kernels.h"

namespace mykfa {
namespace {

constexpr int kCeThreads = 512;
constexpr int kCeWaves = kCeThreads / 64;
constexpr float kLog2e = 1.4426950408889634f;

__device__ inline float wave_max(float x) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) x = fmaxf(x, __shfl_xor(x, m));
    return x;
}

__device__ inline float wave_sum(float x) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m);
    return x;
}

// Reductions over the workgroup; `red` holds one float per wave. The trailing barrier lets the
// caller reuse `red` at once.
__device__ inline float block_max(float x, float* red) {
    x = wave_max(x);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < kCeWaves; ++i) r = fmaxf(r, red[i]);
    __syncthreads();
    return r;
}

__device__ inline float block_sum(float x, float* red) {
    x = wave_sum(x);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < kCeWaves; ++i) r += red[i];
    __syncthreads();
    return r;
}

// e^(x - c) with c pre-multiplied by log2(e): one FMA and the hardware exp2.
__device__ inline float exp_shifted(float x, float c_log2e) { return fast_exp2(fmaf(x, kLog2e, -c_log2e)); }

struct RowHead {
    int64_t target;
    bool ignored, in_range;
};

__device__ inline RowHead row_head(const mykfa_ce_params& p, int64_t row) {
    RowHead h;
    h.target = p.targets[row];
    h.ignored = h.target == (int64_t)p.ignore_index;
    h.in_range = h.target >= 0 && h.target < p.vocab;
    return h;
}

template <typename T>
__device__ inline void zero_row(uint16_t* base, int vocab, bool vec) {
    if (vec) {
        const s16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int c = threadIdx.x * 8; c < vocab; c += kCeThreads * 8) st16(base + c, z);
    } else {
        for (int c = threadIdx.x; c < vocab; c += kCeThreads) base[c] = 0;
    }
}

// Statistics of a row -> (ce, lse) written by lane 0, and the gradient scale factors.
struct RowStats {
    float lse, lse_log2e, softmax_scale;
};

__device__ inline RowStats finish_stats(const mykfa_ce_params& p, int64_t row, const RowHead& h, float m, float s,
                                        float target_logit) {
    RowStats r;
    r.lse = m + logf(s);
    r.lse_log2e = r.lse * kLog2e;
    // d/dlogits [ce + z lse^2] = softmax * (1 + 2 z lse) - onehot (ops/fused_ce.py:59-66)
    r.softmax_scale = p.scale * (1.0f + 2.0f * p.z_coef * r.lse);
    if (threadIdx.x == 0) {
        p.ce[row] = h.in_range ? r.lse - target_logit : __int_as_float(0x7fc00000);  // NaN: no such class
        p.lse[row] = r.lse;
    }
    return r;
}

// bf16 rows keep p = e^(x - max) in the registers that held the logits and form the
// gradient as p * (scale' / sum): one exponential per logit instead of two, and no per-element
// target test -- the lane that holds the target column rewrites that one element after its
// row stores. p lies in [0, 1] and needs no sign, so it is kept in an unsigned 16-bit float
// of this kernel's own: 6 exponent bits (fp32's biased exponents 64..127, i.e. p in
// [2^-63, 1]) and fp32's top 10 mantissa bits, rounded: 11 significant bits, 2^-11 relative,
// over the whole range (fp16 would go subnormal below 2^-14). The gradient, rounded once more
// to bf16, then stays within 0.625 of its ulp. A 16-byte chunk of 8 logits holding any
// p < 2^-63 (x more than ~43.7 below the row max) keeps its logits instead (one flag bit per
// chunk) and recomputes those exponentials from them, as the fp16 rows do for all of theirs.
constexpr uint32_t kKeepBias = 64u << 23;  // fp32 bits of 2^-63, the code 0
constexpr float kKeepMin = 0x1p-63f;

__device__ inline uint32_t keep_code(float p) {  // p in [2^-63, 1] -> 16-bit code
    return (__float_as_uint(p) - kKeepBias + (1u << 12)) >> 13;
}
__device__ inline float keep_value(uint32_t code) { return __uint_as_float((code << 13) + kKeepBias); }

template <typename T, int VPT>
__global__ __launch_bounds__(kCeThreads) void ce_rows_resident_kernel(mykfa_ce_params p) {
    constexpr int NC = VPT / 8;  // 16-byte chunks per lane
    constexpr bool kKeepP = T::code == MYKFA_BF16;
    __shared__ float red[kCeWaves];
    const int64_t row = blockIdx.x;
    uint16_t* base = static_cast<uint16_t*>(p.logits) + row * p.row_stride;
    const RowHead h = row_head(p, row);
    if (h.ignored) {  // uniform across the workgroup
        zero_row<T>(base, p.vocab, true);
        if (threadIdx.x == 0) p.ce[row] = p.lse[row] = 0.f;
        return;
    }
    // The target logit is read before the first barrier, so before any lane overwrites the row.
    const bool owner = kKeepP && h.in_range && (int)((h.target / 8) % kCeThreads) == (int)threadIdx.x;
    const float target_logit = ((threadIdx.x == 0 || owner) && h.in_range) ? T::to_float(base[h.target]) : 0.f;
    s16x8 v[NC];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = (j * kCeThreads + threadIdx.x) * 8;
        if (c < p.vocab) {
            v[j] = ld16(base + c);
#pragma unroll
            for (int i = 0; i < 8; ++i) m = fmaxf(m, T::to_float((uint16_t)v[j][i]));
        }
    }
    m = block_max(m, red);
    const float m_log2e = m * kLog2e;
    float s = 0.f;
    uint32_t raw_mask = 0;  // bit j: chunk j still holds its logits (else the codes of p)
    static_assert(NC <= 32, "one flag bit per chunk");
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = (j * kCeThreads + threadIdx.x) * 8;
        if (c < p.vocab) {
            float e[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                e[i] = exp_shifted(T::to_float((uint16_t)v[j][i]), m_log2e);
                s += e[i];
            }
            if constexpr (kKeepP) {
                float lo = e[0];
#pragma unroll
                for (int i = 1; i < 8; ++i) lo = fminf(lo, e[i]);
                if (lo >= kKeepMin) {
                    uint32_t kw[4];
#pragma unroll
                    for (int i = 0; i < 8; i += 2) kw[i / 2] = keep_code(e[i]) | (keep_code(e[i + 1]) << 16);
                    const u32x4 keep = {kw[0], kw[1], kw[2], kw[3]};
                    v[j] = __builtin_bit_cast(s16x8, keep);
                } else {
                    raw_mask |= 1u << j;  // the chunk keeps its logits
                }
            }
        }
    }
    s = block_sum(s, red);
    const RowStats st = finish_stats(p, row, h, m, s, target_logit);
    if constexpr (kKeepP) {
        const float ratio = st.softmax_scale / s;  // e^(x - lse) * scale' = e^(x - max) * ratio
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int c = (j * kCeThreads + threadIdx.x) * 8;
            if (c < p.vocab) {
                const u32x4 pw = __builtin_bit_cast(u32x4, v[j]);
                uint32_t ow[4];
                if ((raw_mask >> j) & 1u) {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        ow[i] = T::pack2(
                            exp_shifted(T::to_float((uint16_t)(pw[i] & 0xffffu)), st.lse_log2e) * st.softmax_scale,
                            exp_shifted(T::to_float((uint16_t)(pw[i] >> 16)), st.lse_log2e) * st.softmax_scale);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        ow[i] = T::pack2(keep_value(pw[i] & 0xffffu) * ratio, keep_value(pw[i] >> 16) * ratio);
                }
                const u32x4 o = {ow[0], ow[1], ow[2], ow[3]};
                st16(base + c, __builtin_bit_cast(s16x8, o));
            }
        }
        if (owner) {  // after this lane's store of the same 16 bytes
            const float gt = exp_shifted(target_logit, st.lse_log2e) * st.softmax_scale - p.scale;
            base[h.target] = (uint16_t)(T::pack2(gt, 0.f) & 0xffffu);
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = (j * kCeThreads + threadIdx.x) * 8;
        if (c < p.vocab) {
            float g[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                g[i] = exp_shifted(T::to_float((uint16_t)v[j][i]), st.lse_log2e) * st.softmax_scale;
                if (c + i == h.target) g[i] -= p.scale;
            }
            s16x8 o;
#pragma unroll
            for (int i = 0; i < 8; i += 2) {
                const uint32_t w = T::pack2(g[i], g[i + 1]);
                o[i] = (short)(w & 0xffff);
                o[i + 1] = (short)(w >> 16);
            }
            st16(base + c, o);
        }
    }
}

template <typename T>
__global__ __launch_bounds__(kCeThreads) void ce_rows_stream_kernel(mykfa_ce_params p, int vec) {
    __shared__ float red[kCeWaves];
    const int64_t row = blockIdx.x;
    uint16_t* base = static_cast<uint16_t*>(p.logits) + row * p.row_stride;
    const RowHead h = row_head(p, row);
    if (h.ignored) {
        zero_row<T>(base, p.vocab, vec != 0);
        if (threadIdx.x == 0) p.ce[row] = p.lse[row] = 0.f;
        return;
    }
    const float target_logit = (threadIdx.x == 0 && h.in_range) ? T::to_float(base[h.target]) : 0.f;
    // Pass 1: per-lane online max / sum of exponentials, 8 columns at a time.
    float m = -INFINITY, s = 0.f;
    const int step = vec ? kCeThreads * 8 : kCeThreads;
    for (int c = vec ? threadIdx.x * 8 : threadIdx.x; c < p.vocab; c += step) {
        float x[8];
        int n = 1;
        if (vec) {
            const s16x8 raw = ld16(base + c);
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] = T::to_float((uint16_t)raw[i]);
            n = 8;
        } else {
            x[0] = T::to_float(base[c]);
        }
        float cm = x[0];
        for (int i = 1; i < n; ++i) cm = fmaxf(cm, x[i]);
        if (cm > m) {
            s = m == -INFINITY ? 0.f : s * exp_shifted(m, cm * kLog2e);
            m = cm;
        }
        const float m_log2e = m * kLog2e;
        for (int i = 0; i < n; ++i) s += exp_shifted(x[i], m_log2e);
    }
    const float M = block_max(m, red);
    s = m == -INFINITY ? 0.f : s * exp_shifted(m, M * kLog2e);
    s = block_sum(s, red);
    const RowStats st = finish_stats(p, row, h, M, s, target_logit);
    // Pass 2: the gradient, in place.
    for (int c = vec ? threadIdx.x * 8 : threadIdx.x; c < p.vocab; c += step) {
        if (vec) {
            const s16x8 raw = ld16(base + c);
            float g[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                g[i] = exp_shifted(T::to_float((uint16_t)raw[i]), st.lse_log2e) * st.softmax_scale;
                if (c + i == h.target) g[i] -= p.scale;
            }
            s16x8 o;
#pragma unroll
            for (int i = 0; i < 8; i += 2) {
                const uint32_t w = T::pack2(g[i], g[i + 1]);
                o[i] = (short)(w & 0xffff);
                o[i + 1] = (short)(w >> 16);
            }
            st16(base + c, o);
        } else {
            float g = exp_shifted(T::to_float(base[c]), st.lse_log2e) * st.softmax_scale;
            if (c == h.target) g -= p.scale;
            base[c] = T::from_float(g);
        }
    }
}

template <typename T>
hipError_t ce_dtype(const mykfa_ce_params& p, hipStream_t s) {
    const dim3 grid((unsigned)p.rows), block(kCeThreads);
    const bool vec = (p.vocab % 8) == 0 && (p.row_stride % 8) == 0 &&
                     (reinterpret_cast<uintptr_t>(p.logits) & 15) == 0;
    const int per_lane = (p.vocab + kCeThreads - 1) / kCeThreads;
    if (vec && per_lane <= 8) hipLaunchKernelGGL((ce_rows_resident_kernel<T, 8>), grid, block, 0, s, p);
    else if (vec && per_lane <= 16) hipLaunchKernelGGL((ce_rows_resident_kernel<T, 16>), grid, block, 0, s, p);
    else if (vec && per_lane <= 32) hipLaunchKernelGGL((ce_rows_resident_kernel<T, 32>), grid, block, 0, s, p);
    else if (vec && per_lane <= 64) hipLaunchKernelGGL((ce_rows_resident_kernel<T, 64>), grid, block, 0, s, p);
    else if (vec && per_lane <= 128) hipLaunchKernelGGL((ce_rows_resident_kernel<T, 128>), grid, block, 0, s, p);
    else hipLaunchKernelGGL((ce_rows_stream_kernel<T>), grid, block, 0, s, p, vec ? 1 : 0);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_ce_rows(const mykfa_ce_params& p, hipStream_t stream) {
    if (p.dtype == MYKFA_BF16) return ce_dtype<BF16>(p, stream);
    return ce_dtype<FP16>(p, stream);
}

}  // namespace mykfa
