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
// shuffles inside those lanes.
#include "common.h"
#include "kernels.h"

namespace mykfa {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxBwdBlocks = 1024;  // weight-gradient partials: one (2, D) fp32 row per workgroup

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

struct RowPos {
    int64_t tok;  // b * seqlen + s
    int b, s, h;
};

__device__ inline RowPos row_pos(int64_t row, int heads, int seqlen) {
    RowPos r;
    r.tok = row / heads;
    r.h = (int)(row - r.tok * heads);
    r.b = (int)(r.tok / seqlen);
    r.s = (int)(r.tok - (int64_t)r.b * seqlen);
    return r;
}

__device__ inline int64_t clamp_pos(const mykfa_qk_prologue_params& p, int b, int s) {
    int64_t pos = p.position_ids[(int64_t)b * p.pos_batch_stride + (int64_t)s * p.pos_token_stride];
    if (pos < 0) pos = 0;
    if (pos >= p.table_rows) pos = p.table_rows - 1;
    return pos;
}

// ---- prologue forward ------------------------------------------------------------------

template <typename T, int D>
__global__ __launch_bounds__(kThreads) void qk_prologue_fwd_kernel(mykfa_qk_prologue_params p) {
    constexpr int CPR = D / 8;              // 16-byte chunks per row
    constexpr int RPW = kThreads / CPR;     // rows per workgroup pass
    const int c = threadIdx.x % CPR;
    const int heads = p.num_heads + p.num_kv_heads;
    const int64_t rows = (int64_t)p.batch * p.seqlen * heads;
    const bool norm = p.q_weight != nullptr, rope = p.cos != nullptr;
    for (int64_t base = (int64_t)blockIdx.x * RPW; base < rows; base += (int64_t)gridDim.x * RPW) {
        int64_t row = base + threadIdx.x / CPR;
        const bool valid = row < rows;
        if (!valid) row = rows - 1;  // whole lane groups: the shuffles below stay inside valid data
        const RowPos rp = row_pos(row, heads, p.seqlen);
        const bool isq = rp.h < p.num_heads;
        const int hh = isq ? rp.h : rp.h - p.num_heads;
        const uint16_t* src = static_cast<const uint16_t*>(isq ? p.q_in : p.k_in) +
                              (int64_t)rp.b * (isq ? p.qi_batch_stride : p.ki_batch_stride) +
                              (int64_t)rp.s * (isq ? p.qi_token_stride : p.ki_token_stride) +
                              (int64_t)hh * (isq ? p.qi_head_stride : p.ki_head_stride) + c * 8;
        float x[8];
        unpack8<T>(ld16(src), x);
        if (norm) {
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) ss = __fmaf_rn(x[j], x[j], ss);
            ss = row_sum<CPR>(ss);
            const float r = rsqrtf(ss * (1.0f / D) + p.eps);
            float w[8];
            ld8f((isq ? p.q_weight : p.k_weight) + c * 8, w);
            // (x * r) * w in fp32, then the cast of `.to(v.dtype)` (mixers.py:87)
#pragma unroll
            for (int j = 0; j < 8; ++j) x[j] = round_to<T>(__fmul_rn(__fmul_rn(x[j], r), w[j]));
        }
        if (rope) {
            const int64_t pos = clamp_pos(p, rp.b, rp.s);
            float cs[8], sn[8];
            ld8f(p.cos + pos * p.table_stride + c * 8, cs);
            ld8f(p.sin + pos * p.table_stride + c * 8, sn);
            // x*cos + rotate_half(x)*sin, rotate_half(x) = (-x[2i+1], x[2i]) (layers.py:66-70, :97)
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                const float a = x[j], b = x[j + 1];
                x[j] = __fadd_rn(__fmul_rn(a, cs[j]), __fmul_rn(-b, sn[j]));
                x[j + 1] = __fadd_rn(__fmul_rn(b, cs[j + 1]), __fmul_rn(a, sn[j + 1]));
            }
        }
        if (valid) {
            uint16_t* dst = static_cast<uint16_t*>(isq ? p.q_out : p.k_out) +
                            (int64_t)rp.b * (isq ? p.qo_batch_stride : p.ko_batch_stride) +
                            (int64_t)rp.s * (isq ? p.qo_token_stride : p.ko_token_stride) +
                            (int64_t)hh * (isq ? p.qo_head_stride : p.ko_head_stride) + c * 8;
            st16(dst, pack8<T>(x));
        }
    }
}

// ---- prologue backward -----------------------------------------------------------------

template <typename T, int D>
__global__ __launch_bounds__(kThreads) void qk_prologue_bwd_kernel(mykfa_qk_prologue_bwd_params p,
                                                                   float* partial) {
    constexpr int CPR = D / 8;
    constexpr int RPW = kThreads / CPR;
    const mykfa_qk_prologue_params& f = p.fwd;
    const int c = threadIdx.x % CPR, rsub = threadIdx.x / CPR;
    const int heads = f.num_heads + f.num_kv_heads;
    const int64_t rows = (int64_t)f.batch * f.seqlen * heads;
    const bool norm = f.q_weight != nullptr, rope = f.cos != nullptr;
    float wq[8], wk[8];  // this thread's share of the weight gradients (columns 8c..8c+7)
#pragma unroll
    for (int j = 0; j < 8; ++j) wq[j] = wk[j] = 0.f;

    // The q/k rows: their assignment to (workgroup, lane group) depends only on the q/k shape,
    // so the weight-gradient sums do not change with the value-gradient copy below.
    for (int64_t base = (int64_t)blockIdx.x * RPW; base < rows; base += (int64_t)gridDim.x * RPW) {
        int64_t row = base + rsub;
        const bool valid = row < rows;
        if (!valid) row = rows - 1;
        const RowPos rp = row_pos(row, heads, f.seqlen);
        const bool isq = rp.h < f.num_heads;
        const int hh = isq ? rp.h : rp.h - f.num_heads;
        const uint16_t* gsrc = static_cast<const uint16_t*>(isq ? p.dq_out : p.dk_out) +
                               (int64_t)rp.b * (isq ? p.dqo_batch_stride : p.dko_batch_stride) +
                               (int64_t)rp.s * (isq ? p.dqo_token_stride : p.dko_token_stride) +
                               (int64_t)hh * (isq ? p.dqo_head_stride : p.dko_head_stride) + c * 8;
        float g[8];
        unpack8<T>(ld16(gsrc), g);
        if (rope) {
            // Transpose of the rotation: d x[2i] = g[2i] cos[2i] + g[2i+1] sin[2i+1],
            // d x[2i+1] = g[2i+1] cos[2i+1] - g[2i] sin[2i]; then the cast of the gradient of
            // `x.float()` back to the input type.
            const int64_t pos = clamp_pos(f, rp.b, rp.s);
            float cs[8], sn[8];
            ld8f(f.cos + pos * f.table_stride + c * 8, cs);
            ld8f(f.sin + pos * f.table_stride + c * 8, sn);
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                const float a = g[j], b = g[j + 1];
                g[j] = round_to<T>(__fadd_rn(__fmul_rn(a, cs[j]), __fmul_rn(b, sn[j + 1])));
                g[j + 1] = round_to<T>(__fadd_rn(__fmul_rn(b, cs[j + 1]), -__fmul_rn(a, sn[j])));
            }
        }
        if (norm) {
            const uint16_t* xsrc = static_cast<const uint16_t*>(isq ? f.q_in : f.k_in) +
                                   (int64_t)rp.b * (isq ? f.qi_batch_stride : f.ki_batch_stride) +
                                   (int64_t)rp.s * (isq ? f.qi_token_stride : f.ki_token_stride) +
                                   (int64_t)hh * (isq ? f.qi_head_stride : f.ki_head_stride) + c * 8;
            float x[8], w[8];
            unpack8<T>(ld16(xsrc), x);
            ld8f((isq ? f.q_weight : f.k_weight) + c * 8, w);
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) ss = __fmaf_rn(x[j], x[j], ss);
            ss = row_sum<CPR>(ss);
            const float r = rsqrtf(ss * (1.0f / D) + f.eps);
            // y = (x r) w:  dw += g (x r);  gx = g w;  dx = r gx - x r^3 (gx . x) / D
            float dot = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float gx = __fmul_rn(g[j], w[j]);
                if (valid) {
                    if (isq) wq[j] = __fmaf_rn(g[j], __fmul_rn(x[j], r), wq[j]);
                    else wk[j] = __fmaf_rn(g[j], __fmul_rn(x[j], r), wk[j]);
                }
                dot = __fmaf_rn(gx, x[j], dot);
                g[j] = gx;
            }
            dot = row_sum<CPR>(dot);
            const float k3 = dot * r * r * r * (1.0f / D);
#pragma unroll
            for (int j = 0; j < 8; ++j) g[j] = g[j] * r - x[j] * k3;
        }
        if (valid) {
            uint16_t* dst = static_cast<uint16_t*>(isq ? p.dq_in : p.dk_in) +
                            (int64_t)rp.b * (isq ? p.dqi_batch_stride : p.dki_batch_stride) +
                            (int64_t)rp.s * (isq ? p.dqi_token_stride : p.dki_token_stride) +
                            (int64_t)hh * (isq ? p.dqi_head_stride : p.dki_head_stride) + c * 8;
            st16(dst, pack8<T>(g));
        }
    }
    if (p.dv_src != nullptr) {  // the value gradient: a plain 16-byte copy
        const int64_t chunks = (int64_t)f.batch * f.seqlen * f.num_kv_heads * CPR;
        for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < chunks; i += (int64_t)gridDim.x * kThreads) {
            const int cc = (int)(i % CPR);
            const int64_t r = i / CPR;
            const int hh = (int)(r % f.num_kv_heads);
            const int64_t tok = r / f.num_kv_heads;
            const int b = (int)(tok / f.seqlen), sq = (int)(tok % f.seqlen);
            const uint16_t* src = static_cast<const uint16_t*>(p.dv_src) + (int64_t)b * p.dvs_batch_stride +
                                  (int64_t)sq * p.dvs_token_stride + (int64_t)hh * p.dvs_head_stride + cc * 8;
            uint16_t* dst = static_cast<uint16_t*>(p.dv_dst) + (int64_t)b * p.dvd_batch_stride +
                            (int64_t)sq * p.dvd_token_stride + (int64_t)hh * p.dvd_head_stride + cc * 8;
            st16(dst, ld16(src));
        }
    }
    if (!norm) return;  // uniform across the workgroup: no barrier is skipped by part of it

    // Workgroup partial of the weight gradients: sum the RPW row lanes of each column in a
    // fixed order through LDS, one (q, k) row pair of D floats per workgroup.
    __shared__ float red[2][RPW][D];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        red[0][rsub][c * 8 + j] = wq[j];
        red[1][rsub][c * 8 + j] = wk[j];
    }
    __syncthreads();
    for (int t = threadIdx.x; t < 2 * D; t += kThreads) {
        const int which = t / D, col = t % D;
        float s = 0.f;
        for (int r = 0; r < RPW; ++r) s += red[which][r][col];
        partial[((int64_t)blockIdx.x * 2 + which) * D + col] = s;
    }
}

// Fixed-order sum of the per-workgroup partials: (blocks, 2, D) -> dq_weight, dk_weight.
__global__ __launch_bounds__(kThreads) void weight_grad_reduce_kernel(const float* partial, int blocks, int D,
                                                                      float* dq_weight, float* dk_weight) {
    const int t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= 2 * D) return;
    const int which = t / D, col = t % D;
    float s = 0.f;
    for (int b = 0; b < blocks; ++b) s += partial[((int64_t)b * 2 + which) * D + col];
    (which ? dk_weight : dq_weight)[col] = s;
}

// ---- output gate -----------------------------------------------------------------------

__device__ inline float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }

template <typename T>
__global__ __launch_bounds__(kThreads) void gate_fwd_kernel(mykfa_gate_params p) {
    const int cpr = p.width / 8;
    const int64_t total = p.rows * cpr;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total; i += (int64_t)gridDim.x * kThreads) {
        const int64_t r = i / cpr;
        const int c = (int)(i - r * cpr) * 8;
        float x[8], g[8];
        unpack8<T>(ld16(static_cast<const uint16_t*>(p.x) + r * p.x_row_stride + c), x);
        unpack8<T>(ld16(static_cast<const uint16_t*>(p.gate) + r * p.gate_row_stride + c), g);
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = __fmul_rn(x[j], round_to<T>(sigmoid_f32(g[j])));
        st16(static_cast<uint16_t*>(p.y) + r * p.y_row_stride + c, pack8<T>(x));
    }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void gate_bwd_kernel(mykfa_gate_params p) {
    const int cpr = p.width / 8;
    const int64_t total = p.rows * cpr;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total; i += (int64_t)gridDim.x * kThreads) {
        const int64_t r = i / cpr;
        const int c = (int)(i - r * cpr) * 8;
        float x[8], g[8], dy[8], dx[8];
        unpack8<T>(ld16(static_cast<const uint16_t*>(p.x) + r * p.x_row_stride + c), x);
        unpack8<T>(ld16(static_cast<const uint16_t*>(p.gate) + r * p.gate_row_stride + c), g);
        unpack8<T>(ld16(static_cast<const uint16_t*>(p.dy) + r * p.dy_row_stride + c), dy);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float s = round_to<T>(sigmoid_f32(g[j]));
            dx[j] = __fmul_rn(dy[j], s);
            const float ds = round_to<T>(__fmul_rn(dy[j], x[j]));
            g[j] = __fmul_rn(__fmul_rn(ds, 1.0f - s), s);  // sigmoid_backward: g * (1 - s) * s
        }
        st16(static_cast<uint16_t*>(p.dx) + r * p.dx_row_stride + c, pack8<T>(dx));
        st16(static_cast<uint16_t*>(p.dgate) + r * p.dgate_row_stride + c, pack8<T>(g));
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
    const long long rows = (long long)p.batch * p.seqlen * (p.num_heads + p.num_kv_heads);
    hipLaunchKernelGGL((qk_prologue_fwd_kernel<T, D>), dim3(grid_for(rows, rows_per_pass<D>(), 65536)),
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
    hipLaunchKernelGGL((qk_prologue_bwd_kernel<T, D>), dim3(blocks), dim3(kThreads), 0, s, p, ws);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.fwd.q_weight == nullptr) return e;
    hipLaunchKernelGGL(weight_grad_reduce_kernel, dim3((2 * D + kThreads - 1) / kThreads), dim3(kThreads), 0, s,
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
    const long long heads = (long long)num_heads + num_kv_heads;
    const long long rows = (long long)batch * seqlen * heads;
    const long long rpw = kThreads / (head_dim / 8);
    return grid_for(rows, rpw, kMaxBwdBlocks);
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
    const int grid = grid_for(p.rows * (p.width / 8), kThreads, 8192);
    if (p.dtype == MYKFA_BF16) {
        if (backward) hipLaunchKernelGGL(gate_bwd_kernel<BF16>, dim3(grid), dim3(kThreads), 0, stream, p);
        else hipLaunchKernelGGL(gate_fwd_kernel<BF16>, dim3(grid), dim3(kThreads), 0, stream, p);
    } else {
        if (backward) hipLaunchKernelGGL(gate_bwd_kernel<FP16>, dim3(grid), dim3(kThreads), 0, stream, p);
        else hipLaunchKernelGGL(gate_fwd_kernel<FP16>, dim3(grid), dim3(kThreads), 0, stream, p);
    }
    return hipGetLastError();
}

}  // namespace mykfa
