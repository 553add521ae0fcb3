// The attention block's elementwise prologue and epilogue on gfx950:
//   qk_prologue_fwd_kernel  q/k RMSNorm -> cast -> interleaved-pair RoPE -> cast, one pass
//                           (mixers.py:85-89, model/layers.py:22-25, :93-98);
//   qk_prologue_bwd_kernel  its gradient, RMSNorm weight-gradient partials per workgroup and
//                           an optional copy of the value gradient, so one launch writes a
//                           whole fused-projection gradient;
//   weight_grad_reduce_kernel  fixed-order sum of those partials (deterministic);
//   gate_fwd_kernel / gate_bwd_kernel  y = x * sigmoid(gate) and its gradient
//                           (mixers.py:116-117).
// All of them are HBM-bound streams: 16-byte accesses along head_dim, one row of D elements
// per D/8 consecutive lanes, row reductions (sum of squares, the norm's dot product) by lane
// shuffles inside those lanes. Every tensor element is read once, with the non-temporal hint
// (measured with inputs coming from HBM, at cfg3's shape: prologue forward 41.2 -> 33.8 us,
// backward 70.0 -> 60.4, gate forward 39.8 -> 38.9, gate backward 62.5 -> 54.9).
#include "common.h"
#include "kernels.h"

namespace mykfa {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxBwdBlocks = 1024;  // weight-gradient partials: one (2, D) fp32 row per workgroup
constexpr int kHeadsInFlight = 2;     // head rows per lane group whose loads are issued together (measured: 2 > 4 > 8)
constexpr int kBwdHeadsInFlight = 2;  // (two loads per row in the backward; 1 and 4 measured slower)
constexpr int kGateFwdChunks = 1;     // 16-byte chunks per lane per pass (one measured fastest)
constexpr int kGateBwdChunks = 1;

template <typename T>
__device__ inline void unpack8(s16x8 raw, float* f) {
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = T::to_float((uint16_t)raw[j]);
}

template <typename T>
__device__ inline s16x8 pack8(const float* f) {
    s16x8 r;
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        const uint32_t p = T::pack2(f[j], f[j + 1]);
        r[j] = (short)(p & 0xffff);
        r[j + 1] = (short)(p >> 16);
    }
    return r;
}

// Value rounded to the storage type and back (the reference's `.to(dtype)` between ops).
template <typename T>
__device__ inline float round_to(float x) {
    return T::to_float(T::from_float(x));
}

__device__ inline void ld8f(const float* p, float* f) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p);
    const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f[j] = a[j];
        f[4 + j] = b[j];
    }
}

// Sum over the CPR consecutive lanes that hold one row (CPR divides 64, so the xor partners
// stay inside the row's lane group).
template <int CPR>
__device__ inline float row_sum(float x) {
#pragma unroll
    for (int m = CPR / 2; m >= 1; m >>= 1) x += __shfl_xor(x, m);
    return x;
}

__device__ inline int64_t clamp_pos(const mykfa_qk_prologue_params& p, int b, int s) {
    int64_t pos = p.position_ids[(int64_t)b * p.pos_batch_stride + (int64_t)s * p.pos_token_stride];
    if (pos < 0) pos = 0;
    if (pos >= p.table_rows) pos = p.table_rows - 1;
    return pos;
}

// ---- prologue forward ------------------------------------------------------------------

// Work layout of both prologue kernels: one token per lane group of CPR = D/8 lanes (lane c
// holds columns 8c..8c+7 of every row), RPW = 256/CPR tokens per workgroup pass. A lane group
// reads its token's position and cos/sin table row once, then streams the token's Hq q rows
// and Hkv k rows HC at a time, all HC rows' loads issued before any is computed.

template <typename T>
__device__ inline const uint16_t* head_row(const void* base, int64_t bs, int64_t ts, int64_t hs, int b, int s,
                                           int h, int c) {
    return static_cast<const uint16_t*>(base) + (int64_t)b * bs + (int64_t)s * ts + (int64_t)h * hs + c * 8;
}

template <typename T, int D, int HC>
__global__ __launch_bounds__(kThreads) void qk_prologue_fwd_kernel(mykfa_qk_prologue_params p) {
    constexpr int CPR = D / 8;
    constexpr int RPW = kThreads / CPR;
    const int c = threadIdx.x % CPR, lg = threadIdx.x / CPR;
    const int heads = p.num_heads + p.num_kv_heads;
    const int64_t tokens = (int64_t)p.batch * p.seqlen;
    const bool norm = p.q_weight != nullptr, rope = p.cos != nullptr;
    float wq[8], wk[8];  // this lane's 8 columns of the norm weights
    if (norm) {
        ld8f(p.q_weight + c * 8, wq);
        ld8f(p.k_weight + c * 8, wk);
    }
    // the loop bound is uniform within a lane group, so the row shuffles stay inside live lanes
    for (int64_t tok = (int64_t)blockIdx.x * RPW + lg; tok < tokens; tok += (int64_t)gridDim.x * RPW) {
        const int b = (int)(tok / p.seqlen), s = (int)(tok - (int64_t)b * p.seqlen);
        float cs[8], sn[8];
        if (rope) {
            const int64_t pos = clamp_pos(p, b, s);
            ld8f(p.cos + pos * p.table_stride + c * 8, cs);
            ld8f(p.sin + pos * p.table_stride + c * 8, sn);
        }
        for (int h0 = 0; h0 < heads; h0 += HC) {
            float x[HC][8];
#pragma unroll
            for (int u = 0; u < HC; ++u) {
                const int h = min(h0 + u, heads - 1);  // past the last head: an in-bounds reread, not stored
                const bool isq = h < p.num_heads;
                const uint16_t* src = isq ? head_row<T>(p.q_in, p.qi_batch_stride, p.qi_token_stride,
                                                        p.qi_head_stride, b, s, h, c)
                                          : head_row<T>(p.k_in, p.ki_batch_stride, p.ki_token_stride,
                                                        p.ki_head_stride, b, s, h - p.num_heads, c);
                unpack8<T>(ld16_stream(src), x[u]);
            }
#pragma unroll
            for (int u = 0; u < HC; ++u) {
                const int h = h0 + u;
                const bool isq = h < p.num_heads;
                if (norm) {
                    float ss = 0.f;
#pragma unroll
                    for (int j = 0; j < 8; ++j) ss = __fmaf_rn(x[u][j], x[u][j], ss);
                    ss = row_sum<CPR>(ss);
                    const float r = rsqrtf(ss * (1.0f / D) + p.eps);
                    // (x * r) * w in fp32, then the cast of `.to(v.dtype)` (mixers.py:87)
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        x[u][j] = round_to<T>(__fmul_rn(__fmul_rn(x[u][j], r), isq ? wq[j] : wk[j]));
                }
                if (rope) {
                    // x*cos + rotate_half(x)*sin, rotate_half(x) = (-x[2i+1], x[2i]) (layers.py:66-70, :97)
#pragma unroll
                    for (int j = 0; j < 8; j += 2) {
                        const float a = x[u][j], bb = x[u][j + 1];
                        x[u][j] = __fadd_rn(__fmul_rn(a, cs[j]), __fmul_rn(-bb, sn[j]));
                        x[u][j + 1] = __fadd_rn(__fmul_rn(bb, cs[j + 1]), __fmul_rn(a, sn[j + 1]));
                    }
                }
                if (h < heads) {
                    uint16_t* dst = const_cast<uint16_t*>(
                        isq ? head_row<T>(p.q_out, p.qo_batch_stride, p.qo_token_stride, p.qo_head_stride, b, s, h, c)
                            : head_row<T>(p.k_out, p.ko_batch_stride, p.ko_token_stride, p.ko_head_stride, b, s,
                                          h - p.num_heads, c));
                    st16(dst, pack8<T>(x[u]));
                }
            }
        }
    }
}

// ---- prologue backward -----------------------------------------------------------------

template <typename T, int D, int HC>
__global__ __launch_bounds__(kThreads) void qk_prologue_bwd_kernel(mykfa_qk_prologue_bwd_params p,
                                                                   float* partial) {
    constexpr int CPR = D / 8;
    constexpr int RPW = kThreads / CPR;
    const mykfa_qk_prologue_params& f = p.fwd;
    const int c = threadIdx.x % CPR, lg = threadIdx.x / CPR;
    const int heads = f.num_heads + f.num_kv_heads;
    const int64_t tokens = (int64_t)f.batch * f.seqlen;
    const bool norm = f.q_weight != nullptr, rope = f.cos != nullptr;
    float aq[8], ak[8];  // this lane's share of the weight gradients (columns 8c..8c+7)
    float wq[8], wk[8];  // and of the weights
#pragma unroll
    for (int j = 0; j < 8; ++j) aq[j] = ak[j] = 0.f;
    if (norm) {
        ld8f(f.q_weight + c * 8, wq);
        ld8f(f.k_weight + c * 8, wk);
    }
    // The tokens' assignment to (workgroup, lane group) depends only on the q/k shape (the grid
    // is fixed by it), so the weight-gradient sums are the same with or without the value copy.
    for (int64_t tok = (int64_t)blockIdx.x * RPW + lg; tok < tokens; tok += (int64_t)gridDim.x * RPW) {
        const int b = (int)(tok / f.seqlen), s = (int)(tok - (int64_t)b * f.seqlen);
        float cs[8], sn[8];
        if (rope) {
            const int64_t pos = clamp_pos(f, b, s);
            ld8f(f.cos + pos * f.table_stride + c * 8, cs);
            ld8f(f.sin + pos * f.table_stride + c * 8, sn);
        }
        for (int h0 = 0; h0 < heads; h0 += HC) {
            float g[HC][8], x[HC][8];
#pragma unroll
            for (int u = 0; u < HC; ++u) {
                const int h = min(h0 + u, heads - 1);
                const bool isq = h < f.num_heads;
                const uint16_t* gsrc = isq ? head_row<T>(p.dq_out, p.dqo_batch_stride, p.dqo_token_stride,
                                                         p.dqo_head_stride, b, s, h, c)
                                           : head_row<T>(p.dk_out, p.dko_batch_stride, p.dko_token_stride,
                                                         p.dko_head_stride, b, s, h - f.num_heads, c);
                unpack8<T>(ld16_stream(gsrc), g[u]);
                if (norm) {
                    const uint16_t* xsrc = isq ? head_row<T>(f.q_in, f.qi_batch_stride, f.qi_token_stride,
                                                             f.qi_head_stride, b, s, h, c)
                                               : head_row<T>(f.k_in, f.ki_batch_stride, f.ki_token_stride,
                                                             f.ki_head_stride, b, s, h - f.num_heads, c);
                    unpack8<T>(ld16_stream(xsrc), x[u]);
                }
            }
#pragma unroll
            for (int u = 0; u < HC; ++u) {
                const int h = h0 + u;
                const bool isq = h < f.num_heads, live = h < heads;
                if (rope) {
                    // Transpose of the rotation: d x[2i] = g[2i] cos[2i] + g[2i+1] sin[2i+1],
                    // d x[2i+1] = g[2i+1] cos[2i+1] - g[2i] sin[2i]; then the cast of the
                    // gradient of `x.float()` back to the input type.
#pragma unroll
                    for (int j = 0; j < 8; j += 2) {
                        const float a = g[u][j], bb = g[u][j + 1];
                        g[u][j] = round_to<T>(__fadd_rn(__fmul_rn(a, cs[j]), __fmul_rn(bb, sn[j + 1])));
                        g[u][j + 1] = round_to<T>(__fadd_rn(__fmul_rn(bb, cs[j + 1]), -__fmul_rn(a, sn[j])));
                    }
                }
                if (norm) {
                    float ss = 0.f;
#pragma unroll
                    for (int j = 0; j < 8; ++j) ss = __fmaf_rn(x[u][j], x[u][j], ss);
                    ss = row_sum<CPR>(ss);
                    const float r = rsqrtf(ss * (1.0f / D) + f.eps);
                    // y = (x r) w:  dw += g (x r);  gx = g w;  dx = r gx - x r^3 (gx . x) / D
                    float dot = 0.f;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const float gx = __fmul_rn(g[u][j], isq ? wq[j] : wk[j]);
                        const float contrib = live ? g[u][j] * __fmul_rn(x[u][j], r) : 0.f;
                        if (isq) aq[j] += contrib;
                        else ak[j] += contrib;
                        dot = __fmaf_rn(gx, x[u][j], dot);
                        g[u][j] = gx;
                    }
                    dot = row_sum<CPR>(dot);
                    const float k3 = dot * r * r * r * (1.0f / D);
#pragma unroll
                    for (int j = 0; j < 8; ++j) g[u][j] = g[u][j] * r - x[u][j] * k3;
                }
                if (live) {
                    uint16_t* dst = const_cast<uint16_t*>(
                        isq ? head_row<T>(p.dq_in, p.dqi_batch_stride, p.dqi_token_stride, p.dqi_head_stride, b, s,
                                          h, c)
                            : head_row<T>(p.dk_in, p.dki_batch_stride, p.dki_token_stride, p.dki_head_stride, b, s,
                                          h - f.num_heads, c));
                    st16(dst, pack8<T>(g[u]));
                }
            }
        }
    }
    if (p.dv_src != nullptr) {  // the value gradient: a plain 16-byte copy, 4 chunks per lane in flight
        const int64_t chunks = (int64_t)f.batch * f.seqlen * f.num_kv_heads * CPR;
        for (int64_t i0 = (int64_t)blockIdx.x * kThreads * 4 + threadIdx.x; i0 < chunks;
             i0 += (int64_t)gridDim.x * kThreads * 4) {
            s16x8 v[4];
            const uint16_t* src[4];
            uint16_t* dst[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                int64_t i = i0 + (int64_t)u * kThreads;
                if (i >= chunks) i = chunks - 1;  // in-bounds reread; not stored
                const int cc = (int)(i % CPR);
                const int64_t r = i / CPR;
                const int hh = (int)(r % f.num_kv_heads);
                const int64_t tk = r / f.num_kv_heads;
                const int b = (int)(tk / f.seqlen), sq = (int)(tk % f.seqlen);
                src[u] = head_row<T>(p.dv_src, p.dvs_batch_stride, p.dvs_token_stride, p.dvs_head_stride, b, sq, hh, cc);
                dst[u] = const_cast<uint16_t*>(
                    head_row<T>(p.dv_dst, p.dvd_batch_stride, p.dvd_token_stride, p.dvd_head_stride, b, sq, hh, cc));
                v[u] = ld16_stream(src[u]);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (i0 + (int64_t)u * kThreads < chunks) st16(dst[u], v[u]);
        }
    }
    if (!norm) return;  // uniform across the workgroup: no barrier is skipped by part of it

    // Workgroup partial of the weight gradients: sum the RPW lane groups of each column in a
    // fixed order through LDS, one (q, k) row pair of D floats per workgroup.
    __shared__ float red[2][RPW][D];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        red[0][lg][c * 8 + j] = aq[j];
        red[1][lg][c * 8 + j] = ak[j];
    }
    __syncthreads();
    for (int t = threadIdx.x; t < 2 * D; t += kThreads) {
        const int which = t / D, col = t % D;
        float sum = 0.f;
        for (int r = 0; r < RPW; ++r) sum += red[which][r][col];
        partial[((int64_t)blockIdx.x * 2 + which) * D + col] = sum;
    }
}

// Fixed-order sum of the per-workgroup partials, laid out (blocks, 2 * D): column g < D is
// dq_weight[g], g >= D dk_weight[g - D]. A workgroup owns kRedCols columns; its kRedSlices
// lane slices each sum every kRedSlices-th partial row (independent loads in flight), then
// the slices are added in slice order through LDS. Four columns per workgroup: 2 D / 4
// workgroups, 64 slices, so a slice has few dependent load rounds (cfg3's prologue backward with
// the sum: 60.9 -> 58.3 us against 16 columns).
constexpr int kRedCols = 4, kRedSlices = kThreads / kRedCols;

__global__ __launch_bounds__(kThreads) void weight_grad_reduce_kernel(const float* partial, int blocks, int D,
                                                                      float* dq_weight, float* dk_weight) {
    __shared__ float red[kRedSlices][kRedCols];
    const int cl = threadIdx.x % kRedCols, slice = threadIdx.x / kRedCols;
    const int g = blockIdx.x * kRedCols + cl;  // 2 * D is a multiple of kRedCols for every head_dim
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    int b = slice;
    for (; b + 3 * kRedSlices < blocks; b += 4 * kRedSlices) {
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[u] += partial[(int64_t)(b + u * kRedSlices) * 2 * D + g];
    }
    for (; b < blocks; b += kRedSlices) acc[0] += partial[(int64_t)b * 2 * D + g];
    red[slice][cl] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    __syncthreads();
    if (slice == 0) {
        float sum = 0.f;
        for (int r = 0; r < kRedSlices; ++r) sum += red[r][cl];
        if (g < D) dq_weight[g] = sum;
        else dk_weight[g - D] = sum;
    }
}

// ---- output gate -----------------------------------------------------------------------

__device__ inline float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }

// U 16-byte chunks per lane per pass (chunk i = pass base + u * kThreads + lane: coalesced),
// all loads issued before any chunk is computed.
template <typename T, int U>
__global__ __launch_bounds__(kThreads) void gate_fwd_kernel(mykfa_gate_params p) {
    const int cpr = p.width / 8;
    const int64_t total = p.rows * cpr;
    for (int64_t base = (int64_t)blockIdx.x * kThreads * U + threadIdx.x; base < total;
         base += (int64_t)gridDim.x * kThreads * U) {
        float x[U][8], g[U][8];
        int64_t r[U];
        int c[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            int64_t i = base + (int64_t)u * kThreads;
            if (i >= total) i = total - 1;  // in-bounds reread; the store below is skipped
            r[u] = i / cpr;
            c[u] = (int)(i - r[u] * cpr) * 8;
            unpack8<T>(ld16_stream(static_cast<const uint16_t*>(p.x) + r[u] * p.x_row_stride + c[u]), x[u]);
            unpack8<T>(ld16_stream(static_cast<const uint16_t*>(p.gate) + r[u] * p.gate_row_stride + c[u]), g[u]);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int j = 0; j < 8; ++j) x[u][j] = __fmul_rn(x[u][j], round_to<T>(sigmoid_f32(g[u][j])));
            if (base + (int64_t)u * kThreads < total)
                st16(static_cast<uint16_t*>(p.y) + r[u] * p.y_row_stride + c[u], pack8<T>(x[u]));
        }
    }
}

template <typename T, int U>
__global__ __launch_bounds__(kThreads) void gate_bwd_kernel(mykfa_gate_params p) {
    const int cpr = p.width / 8;
    const int64_t total = p.rows * cpr;
    for (int64_t base = (int64_t)blockIdx.x * kThreads * U + threadIdx.x; base < total;
         base += (int64_t)gridDim.x * kThreads * U) {
        float x[U][8], g[U][8], dy[U][8];
        int64_t r[U];
        int c[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            int64_t i = base + (int64_t)u * kThreads;
            if (i >= total) i = total - 1;
            r[u] = i / cpr;
            c[u] = (int)(i - r[u] * cpr) * 8;
            unpack8<T>(ld16_stream(static_cast<const uint16_t*>(p.x) + r[u] * p.x_row_stride + c[u]), x[u]);
            unpack8<T>(ld16_stream(static_cast<const uint16_t*>(p.gate) + r[u] * p.gate_row_stride + c[u]), g[u]);
            unpack8<T>(ld16_stream(static_cast<const uint16_t*>(p.dy) + r[u] * p.dy_row_stride + c[u]), dy[u]);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float dx[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float sg = round_to<T>(sigmoid_f32(g[u][j]));
                dx[j] = __fmul_rn(dy[u][j], sg);
                const float ds = round_to<T>(__fmul_rn(dy[u][j], x[u][j]));
                g[u][j] = __fmul_rn(__fmul_rn(ds, 1.0f - sg), sg);  // sigmoid_backward: g (1 - s) s
            }
            if (base + (int64_t)u * kThreads < total) {
                st16(static_cast<uint16_t*>(p.dx) + r[u] * p.dx_row_stride + c[u], pack8<T>(dx));
                st16(static_cast<uint16_t*>(p.dgate) + r[u] * p.dgate_row_stride + c[u], pack8<T>(g[u]));
            }
        }
    }
}

template <int D>
int rows_per_pass() { return kThreads / (D / 8); }

int grid_for(long long items, long long per_block, long long cap) {
    long long g = (items + per_block - 1) / per_block;
    if (g > cap) g = cap;
    return (int)(g < 1 ? 1 : g);
}

template <typename T, int D>
hipError_t prologue_fwd_d(const mykfa_qk_prologue_params& p, hipStream_t s) {
    const long long tokens = (long long)p.batch * p.seqlen;
    hipLaunchKernelGGL((qk_prologue_fwd_kernel<T, D, kHeadsInFlight>), dim3(grid_for(tokens, rows_per_pass<D>(), 65536)),
                       dim3(kThreads), 0, s, p);
    return hipGetLastError();
}

template <typename T>
hipError_t prologue_fwd_t(const mykfa_qk_prologue_params& p, hipStream_t s) {
    switch (p.head_dim) {
        case 16: return prologue_fwd_d<T, 16>(p, s);
        case 32: return prologue_fwd_d<T, 32>(p, s);
        case 64: return prologue_fwd_d<T, 64>(p, s);
        case 128: return prologue_fwd_d<T, 128>(p, s);
        default: return prologue_fwd_d<T, 256>(p, s);
    }
}

template <typename T, int D>
hipError_t prologue_bwd_d(const mykfa_qk_prologue_bwd_params& p, float* ws, hipStream_t s) {
    const int blocks = qk_prologue_bwd_blocks(p.fwd.batch, p.fwd.seqlen, p.fwd.num_heads, p.fwd.num_kv_heads,
                                              p.fwd.head_dim);
    hipLaunchKernelGGL((qk_prologue_bwd_kernel<T, D, kBwdHeadsInFlight>), dim3(blocks), dim3(kThreads), 0, s, p, ws);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.fwd.q_weight == nullptr) return e;
    hipLaunchKernelGGL(weight_grad_reduce_kernel, dim3(2 * D / kRedCols), dim3(kThreads), 0, s,
                       (const float*)ws, blocks, D, p.dq_weight, p.dk_weight);
    return hipGetLastError();
}

template <typename T>
hipError_t prologue_bwd_t(const mykfa_qk_prologue_bwd_params& p, float* ws, hipStream_t s) {
    switch (p.fwd.head_dim) {
        case 16: return prologue_bwd_d<T, 16>(p, ws, s);
        case 32: return prologue_bwd_d<T, 32>(p, ws, s);
        case 64: return prologue_bwd_d<T, 64>(p, ws, s);
        case 128: return prologue_bwd_d<T, 128>(p, ws, s);
        default: return prologue_bwd_d<T, 256>(p, ws, s);
    }
}

}  // namespace

int qk_prologue_bwd_blocks(int batch, int seqlen, int num_heads, int num_kv_heads, int head_dim) {
    (void)num_heads;
    (void)num_kv_heads;
    const long long tokens = (long long)batch * seqlen;
    return grid_for(tokens, kThreads / (head_dim / 8), kMaxBwdBlocks);
}

size_t qk_prologue_bwd_workspace_bytes(int batch, int seqlen, int num_heads, int num_kv_heads, int head_dim) {
    const int blocks = qk_prologue_bwd_blocks(batch, seqlen, num_heads, num_kv_heads, head_dim);
    return (size_t)blocks * 2 * head_dim * sizeof(float);
}

hipError_t launch_qk_prologue_fwd(const mykfa_qk_prologue_params& p, hipStream_t stream) {
    if (p.dtype == MYKFA_BF16) return prologue_fwd_t<BF16>(p, stream);
    return prologue_fwd_t<FP16>(p, stream);
}

hipError_t launch_qk_prologue_bwd(const mykfa_qk_prologue_bwd_params& p, void* ws, hipStream_t stream) {
    if (p.fwd.dtype == MYKFA_BF16) return prologue_bwd_t<BF16>(p, static_cast<float*>(ws), stream);
    return prologue_bwd_t<FP16>(p, static_cast<float*>(ws), stream);
}

hipError_t launch_gate(const mykfa_gate_params& p, bool backward, hipStream_t stream) {
    const long long chunks = p.rows * (p.width / 8);
    if (backward) {
        const int grid = grid_for(chunks, (long long)kThreads * kGateBwdChunks, 8192);
        if (p.dtype == MYKFA_BF16)
            hipLaunchKernelGGL((gate_bwd_kernel<BF16, kGateBwdChunks>), dim3(grid), dim3(kThreads), 0, stream, p);
        else
            hipLaunchKernelGGL((gate_bwd_kernel<FP16, kGateBwdChunks>), dim3(grid), dim3(kThreads), 0, stream, p);
    } else {
        const int grid = grid_for(chunks, (long long)kThreads * kGateFwdChunks, 8192);
        if (p.dtype == MYKFA_BF16)
            hipLaunchKernelGGL((gate_fwd_kernel<BF16, kGateFwdChunks>), dim3(grid), dim3(kThreads), 0, stream, p);
        else
            hipLaunchKernelGGL((gate_fwd_kernel<FP16, kGateFwdChunks>), dim3(grid), dim3(kThreads), 0, stream, p);
    }
    return hipGetLastError();
}

}  // namespace mykfa
