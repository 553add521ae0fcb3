// KV-cache decode: split-K forward over the cache length plus an LSE merge, and the KV
// append (replaces the decode configuration of _fwd_kernel, flash_attn.py:324, :364, and
// the cache writes of flash_attn_with_kvcache, flash_attn.py:480-488).
//
// Rows. All GROUP query heads of one KV head and all seqlen_q queries are packed as the
// rows of one 16-row MFMA tile (row = head_in_group * seqlen_q + query), so each K/V byte
// is read from HBM once per GQA group, not once per query head. With GROUP = 4 and the
// 4-query MTP draft this exactly fills the tile.
//
// Split-K. Workgroup (split, batch, kv-head-and-row-tile) covers the keys
// [split * chunk, (split + 1) * chunk) of its sequence; its 4 waves take interleaved 32-key
// tiles. Per tile a wave computes S^T = K Q^T (16x16x32 MFMA, K loaded from HBM straight
// into A-operand registers, one tile ahead), runs the online softmax, and accumulates
// O^T += V^T P^T with V staged in wave-private LDS and read back transposed. The waves
// merge through LDS; a workgroup then writes either the final O/LSE (one split) or an fp32
// partial (O, lse) that the merge kernel combines: lse = log2(sum_s 2^lse_s),
// O = sum_s 2^(lse_s - lse) O_s.
#include "common.h"
#include "kernels.h"

namespace mykfa {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kTile = 32;  // keys per wave step

struct DecodeArgs {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    uint16_t* o;
    float* lse;
    int64_t qbs, qts, qhs, kbs, kts, khs, vbs, vts, vhs, obs, ots, ohs, lse_hs;
    const int32_t* seqused_k;
    int nq;        // queries per sequence
    int cap;       // keys per sequence when seqused_k is NULL (the cache capacity)
    int wl, wr;
    float qk_scale;
    int group;
    int rows;      // group * nq
    int row_tiles; // ceil(rows / 16)
    int num_heads;
    int chunk;     // keys per split (multiple of kTile)
    int splits;
    float* ws_o;   // [splits][batch][num_heads][nq][D]
    float* ws_lse; // [splits][batch][num_heads][nq]
    int batch;
};

// Keys of sequence b, clamped to the cache capacity so no read leaves the cache.
__device__ inline int seq_keys(const DecodeArgs& a, int b) {
    if (!a.seqused_k) return a.cap;
    const int L = a.seqused_k[b];
    return L < 0 ? 0 : (L > a.cap ? a.cap : L);
}

// Keys any row of sequence b can see, as a kTile-aligned [lo, hi) (flash_attn.py:58-68 with
// the queries as the self block).
__device__ inline Ranges decode_ranges(const DecodeArgs& a, int L) {
    const int lo_off = band_lo(L, a.nq, a.wl), hi_off = band_hi(L, a.nq, a.wr);
    return block_ranges(0, a.nq, lo_off, hi_off, L, kTile);
}

template <int D, typename T>
__global__ __launch_bounds__(kThreads) void decode_splitk_kernel(DecodeArgs a) {
    constexpr int KD = D < 32 ? 1 : D / 32;  // 32-wide d steps of S^T (D = 16 pads to 32)
    constexpr int DB = (D + 15) / 16;        // 16-row blocks of O^T
    constexpr int VPL = (kTile * D / 8 + 63) / 64;  // 16-byte V chunks per lane per tile
    __shared__ __attribute__((aligned(16))) uint16_t vlds[kWaves][kTile * D];
    __shared__ float red_m[kWaves][16], red_l[kWaves][16];
    __shared__ float red_o[kWaves][16][D + 1];

    const int split = blockIdx.x, b = blockIdx.y;
    const int kvh = blockIdx.z / a.row_tiles, rt = blockIdx.z % a.row_tiles;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int l16 = lane & 15, G = lane >> 4;

    const int L = seq_keys(a, b);
    const Ranges rg = decode_ranges(a, L);
    int k0 = split * a.chunk, k1 = k0 + a.chunk;
    k0 = k0 > rg.lo ? k0 : rg.lo;
    k1 = k1 < rg.hi ? k1 : rg.hi;
    if (a.splits > 1 && k0 >= k1) return;  // this split holds no visible key: the merge skips it

    const int lo_off = band_lo(L, a.nq, a.wl), hi_off = band_hi(L, a.nq, a.wr);

    // Q^T operand: lane holds Q[row l16][32 kk + 8 G + i].
    const int row = rt * 16 + l16;
    const bool row_ok = row < a.rows;
    const int gh = row_ok ? row / a.nq : 0, qi = row_ok ? row % a.nq : 0;
    const int h = kvh * a.group + gh;
    s16x8 qop[KD];
    {
        const uint16_t* qp = a.q + (int64_t)b * a.qbs + (int64_t)qi * a.qts + (int64_t)h * a.qhs;
#pragma unroll
        for (int kk = 0; kk < KD; ++kk) {
            s16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
            const int d0 = 32 * kk + 8 * G;
            if (row_ok && d0 < D) v = ld16(qp + d0);
            qop[kk] = v;
        }
    }

    const uint16_t* kbase = a.k + (int64_t)b * a.kbs + (int64_t)kvh * a.khs;
    const uint16_t* vbase = a.v + (int64_t)b * a.vbs + (int64_t)kvh * a.vhs;
    uint16_t* vs = vlds[wave];

    f32x4 acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_i = kNegFloor, l_i = 0.f;

    // One tile of registers: K in A-operand order (two 16-key blocks), V as row chunks.
    struct TileRegs {
        s16x8 k[2][KD];
        s16x8 v[VPL];
    };
    auto load_tile = [&](int t0, TileRegs& tr) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            // Block kb of the tile holds keys t0 + 8 (rho / 4) + 4 kb + rho % 4 in its rows.
            const int key = t0 + 8 * (l16 >> 2) + 4 * kb + (l16 & 3);
#pragma unroll
            for (int kk = 0; kk < KD; ++kk) {
                s16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
                const int d0 = 32 * kk + 8 * G;
                if (key < L && d0 < D) v = ld16(kbase + (int64_t)key * a.kts + d0);
                tr.k[kb][kk] = v;
            }
        }
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int idx = lane + 64 * i;
            const int r = idx / (D / 8), ch = idx % (D / 8);
            s16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
            if (idx < kTile * D / 8 && t0 + r < L) v = ld16(vbase + (int64_t)(t0 + r) * a.vts + ch * 8);
            tr.v[i] = v;
        }
    };
    auto compute_tile = [&](int t0, const TileRegs& tr) {
        // Stage this tile's V rows in wave-private LDS (swizzled) for the transpose read.
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int idx = lane + 64 * i;
            if (idx < kTile * D / 8) {
                const int r = idx / (D / 8), ch = idx % (D / 8);
                *reinterpret_cast<s16x8*>(vs + r * D + ((ch ^ lds_swz<D>(r)) << 3)) = tr.v[i];
            }
        }
        // S^T = K Q^T for the two 16-key blocks of the tile.
        f32x4 st[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            st[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < KD; ++kk) st[kb] = T::mfma16(tr.k[kb][kk], qop[kk], st[kb]);
        }
        const bool masked = !(t0 >= rg.mid_lo && t0 + kTile <= rg.mid_hi);
        float mx = kNegFloor;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float x = st[kb][r] * a.qk_scale;
                if (masked) {
                    const int key = t0 + 8 * G + 4 * kb + r;
                    const int rel = key - qi;
                    x = (rel >= lo_off && rel <= hi_off && key < L) ? x : -INFINITY;
                }
                st[kb][r] = x;
                mx = fmaxf(mx, x);
            }
        // Row max across the 4 lane groups holding this row (lanes l16 + 16 G).
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_i, mx);
        const float alpha = fast_exp2(m_i - m_new);
        float p[8];
        float lsum = 0.f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                p[4 * kb + r] = fast_exp2(st[kb][r] - m_new);
                lsum += p[4 * kb + r];
            }
        l_i = l_i * alpha + lsum;
        m_i = m_new;
        u32x4 pw = {T::pack2(p[0], p[1]), T::pack2(p[2], p[3]), T::pack2(p[4], p[5]), T::pack2(p[6], p[7])};
        const s16x8 pop = __builtin_bit_cast(s16x8, pw);
        // O^T += V^T P^T: A operand V[8G + i][16 db + l16] through the transpose read.
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            acc[db] *= alpha;
            const int vrow = 8 * G + (l16 >> 2);
            const int col = 16 * db + 4 * (l16 & 3);
            s16x4 lo4 = ds_read_tr(vs + lds_off<D>(vrow, col));
            s16x4 hi4 = ds_read_tr(vs + lds_off<D>(vrow + 4, col));
            acc[db] = T::mfma16(cat4(lo4, hi4), pop, acc[db]);
        }
    };

    // Two register tiles in flight: the next tile's loads overlap this tile's math.
    const int step = kWaves * kTile;
    TileRegs ta, tb;
    int t0 = k0 + wave * kTile;
    if (t0 < k1) load_tile(t0, ta);
    for (; t0 < k1; t0 += 2 * step) {
        const int t1 = t0 + step;
        if (t1 < k1) load_tile(t1, tb);
        compute_tile(t0, ta);
        if (t1 >= k1) break;
        if (t1 + step < k1) load_tile(t1 + step, ta);
        compute_tile(t1, tb);
    }

    // Merge the 4 waves: row stats per lane group are partial sums over that group's keys.
    float l_row = l_i;
    l_row += __shfl_xor(l_row, 16);
    l_row += __shfl_xor(l_row, 32);
    if (G == 0) {
        red_m[wave][l16] = m_i;
        red_l[wave][l16] = l_row;
    }
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int d = 16 * db + 4 * G + r;
            if (d < D) red_o[wave][l16][d] = acc[db][r];
        }
    __syncthreads();
    // Each thread finalizes (row, d) pairs of the tile.
    for (int idx = tid; idx < 16 * D; idx += kThreads) {
        const int rr = idx / D, d = idx % D;
        const int grow = rt * 16 + rr;
        if (grow >= a.rows) continue;
        float M = kNegFloor;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, red_m[w][rr]);
        float lt = 0.f, ot = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float s = fast_exp2(red_m[w][rr] - M);
            lt += red_l[w][rr] * s;
            ot += red_o[w][rr][d] * s;
        }
        const int hh = kvh * a.group + grow / a.nq, qq = grow % a.nq;
        if (a.splits == 1) {
            // Final output (flash_attn.py:147-154).
            const bool empty = lt == 0.f;
            const float val = empty ? 0.f : ot / lt;
            a.o[(int64_t)b * a.obs + (int64_t)qq * a.ots + (int64_t)hh * a.ohs + d] = T::from_float(val);
            if (d == 0)
                a.lse[(int64_t)hh * a.lse_hs + (int64_t)b * a.nq + qq] = empty ? INFINITY : M + fast_log2(lt);
        } else {
            // Normalized partial: O_s = ot / lt, lse_s = M + log2(lt) (-inf when empty).
            const int64_t prow = (((int64_t)split * a.batch + b) * a.num_heads + hh) * a.nq + qq;
            const bool empty = lt == 0.f;
            a.ws_o[prow * D + d] = empty ? 0.f : ot / lt;
            if (d == 0) a.ws_lse[prow] = empty ? -INFINITY : M + fast_log2(lt);
        }
    }
}

// One wave per output row (batch, head, query): combines the splits that hold visible keys.
template <int D, typename T>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t rowid = (int64_t)blockIdx.x * 4 + wave;  // over batch * num_heads * nq
    const int64_t total = (int64_t)a.batch * a.num_heads * a.nq;
    if (rowid >= total) return;
    const int qq = rowid % a.nq;
    const int hh = (rowid / a.nq) % a.num_heads;
    const int b = rowid / ((int64_t)a.nq * a.num_heads);
    const int L = seq_keys(a, b);
    const Ranges rg = decode_ranges(a, L);
    int s_lo = rg.lo / a.chunk, s_hi = rg.hi > rg.lo ? (rg.hi - 1) / a.chunk + 1 : s_lo;
    if (s_hi > a.splits) s_hi = a.splits;
    const int64_t rstride = (int64_t)a.batch * a.num_heads * a.nq;
    const int64_t base = ((int64_t)b * a.num_heads + hh) * a.nq + qq;
    float M = -INFINITY;
    for (int s = s_lo; s < s_hi; ++s) M = fmaxf(M, a.ws_lse[s * rstride + base]);
    constexpr int PER = (D + 63) / 64;
    float o[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) o[i] = 0.f;
    float lsum = 0.f;
    if (M != -INFINITY) {
        for (int s = s_lo; s < s_hi; ++s) {
            const float ls = a.ws_lse[s * rstride + base];
            const float w = fast_exp2(ls - M);  // 0 for empty splits (ls = -inf)
            lsum += w;
            const float* op = a.ws_o + (s * rstride + base) * D;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int d = lane + 64 * i;
                if (d < D) o[i] += w * op[d];
            }
        }
    }
    const bool empty = M == -INFINITY;
    const float inv = empty ? 0.f : 1.f / lsum;
    uint16_t* out = a.o + (int64_t)b * a.obs + (int64_t)qq * a.ots + (int64_t)hh * a.ohs;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int d = lane + 64 * i;
        if (d < D) out[d] = T::from_float(o[i] * inv);
    }
    if (lane == 0) a.lse[(int64_t)hh * a.lse_hs + (int64_t)b * a.nq + qq] = empty ? INFINITY : M + fast_log2(lsum);
}

DecodeArgs make_args(const mykfa_decode_params& p, int splits, void* ws) {
    const mykfa_fwd_params& f = p.fwd;
    DecodeArgs a;
    a.q = static_cast<const uint16_t*>(f.q);
    a.k = static_cast<const uint16_t*>(f.k);
    a.v = static_cast<const uint16_t*>(f.v);
    a.o = static_cast<uint16_t*>(f.o);
    a.lse = f.lse;
    a.qbs = f.q_batch_stride; a.qts = f.q_token_stride; a.qhs = f.q_head_stride;
    a.kbs = f.k_batch_stride; a.kts = f.k_token_stride; a.khs = f.k_head_stride;
    a.vbs = f.v_batch_stride; a.vts = f.v_token_stride; a.vhs = f.v_head_stride;
    a.obs = f.o_batch_stride; a.ots = f.o_token_stride; a.ohs = f.o_head_stride;
    a.lse_hs = f.lse_head_stride;
    a.seqused_k = f.seqused_k;
    a.nq = f.max_seqlen_q;
    a.cap = f.max_seqlen_k;
    a.wl = f.window_left;
    a.wr = f.window_right;
    a.qk_scale = f.softmax_scale * 1.4426950408889634f;
    a.group = f.num_heads / f.num_kv_heads;
    a.rows = a.group * a.nq;
    a.row_tiles = (a.rows + 15) / 16;
    a.num_heads = f.num_heads;
    a.splits = splits;
    int chunk = (f.max_seqlen_k + splits - 1) / splits;
    chunk = (chunk + kTile - 1) / kTile * kTile;
    a.chunk = chunk > 0 ? chunk : kTile;
    a.batch = f.batch;
    const size_t rows_total = (size_t)f.batch * f.num_heads * f.max_seqlen_q;
    a.ws_o = static_cast<float*>(ws);
    a.ws_lse = ws ? a.ws_o + (size_t)splits * rows_total * f.head_dim : nullptr;
    return a;
}

template <typename T>
hipError_t splitk_dtype(const DecodeArgs& a, int D, int num_kv_heads, hipStream_t s) {
    dim3 grid(a.splits, a.batch, num_kv_heads * a.row_tiles);
    switch (D) {
        case 16: hipLaunchKernelGGL((decode_splitk_kernel<16, T>), grid, dim3(kThreads), 0, s, a); break;
        case 32: hipLaunchKernelGGL((decode_splitk_kernel<32, T>), grid, dim3(kThreads), 0, s, a); break;
        case 64: hipLaunchKernelGGL((decode_splitk_kernel<64, T>), grid, dim3(kThreads), 0, s, a); break;
        case 128: hipLaunchKernelGGL((decode_splitk_kernel<128, T>), grid, dim3(kThreads), 0, s, a); break;
        case 256: hipLaunchKernelGGL((decode_splitk_kernel<256, T>), grid, dim3(kThreads), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <typename T>
hipError_t merge_dtype(const DecodeArgs& a, int D, hipStream_t s) {
    const int64_t rows = (int64_t)a.batch * a.num_heads * a.nq;
    dim3 grid((unsigned)((rows + 3) / 4));
    switch (D) {
        case 16: hipLaunchKernelGGL((decode_merge_kernel<16, T>), grid, dim3(256), 0, s, a); break;
        case 32: hipLaunchKernelGGL((decode_merge_kernel<32, T>), grid, dim3(256), 0, s, a); break;
        case 64: hipLaunchKernelGGL((decode_merge_kernel<64, T>), grid, dim3(256), 0, s, a); break;
        case 128: hipLaunchKernelGGL((decode_merge_kernel<128, T>), grid, dim3(256), 0, s, a); break;
        case 256: hipLaunchKernelGGL((decode_merge_kernel<256, T>), grid, dim3(256), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- KV append --------------------------------------------------------------------------

__global__ __launch_bounds__(256) void kv_append_kernel(mykfa_kv_append_params p) {
    const int cpr = p.head_dim / 8;
    const int64_t per_tok = (int64_t)p.num_kv_heads * cpr;
    const int64_t total = (int64_t)p.batch * p.seqlen_new * per_tok;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int ch = idx % cpr;
        const int hh = (idx / cpr) % p.num_kv_heads;
        const int t = (idx / per_tok) % p.seqlen_new;
        const int b = idx / (per_tok * p.seqlen_new);
        const int pos = p.cache_seqlens[b] + t;
        if (pos < 0 || pos >= p.capacity) continue;  // outside the cache: nothing to write
        const uint16_t* kn = static_cast<const uint16_t*>(p.k_new) + (int64_t)b * p.kn_batch_stride +
                             (int64_t)t * p.kn_token_stride + (int64_t)hh * p.kn_head_stride + ch * 8;
        const uint16_t* vn = static_cast<const uint16_t*>(p.v_new) + (int64_t)b * p.vn_batch_stride +
                             (int64_t)t * p.vn_token_stride + (int64_t)hh * p.vn_head_stride + ch * 8;
        uint16_t* kc = static_cast<uint16_t*>(p.k_cache) + (int64_t)b * p.kc_batch_stride +
                       (int64_t)pos * p.kc_token_stride + (int64_t)hh * p.kc_head_stride + ch * 8;
        uint16_t* vc = static_cast<uint16_t*>(p.v_cache) + (int64_t)b * p.vc_batch_stride +
                       (int64_t)pos * p.vc_token_stride + (int64_t)hh * p.vc_head_stride + ch * 8;
        st16(kc, ld16(kn));
        st16(vc, ld16(vn));
    }
}

}  // namespace

size_t decode_workspace_bytes(int batch, int num_heads, int seqlen_q, int head_dim, int num_splits) {
    if (num_splits <= 1) return 0;
    const size_t rows = (size_t)batch * num_heads * seqlen_q;
    return (size_t)num_splits * rows * ((size_t)head_dim + 1) * sizeof(float);
}

int decode_default_splits(int batch, int num_kv_heads, int capacity) {
    // Aim for about 16 workgroups per CU on the 256-CU chip if every cache were full, with at
    // least 256 keys per split; caches are usually partly filled, so this keeps several
    // workgroups per CU in flight for typical fills.
    const long long target = 256LL * 16;
    const long long pairs = (long long)(batch > 0 ? batch : 1) * (num_kv_heads > 0 ? num_kv_heads : 1);
    long long splits = (target + pairs - 1) / pairs;
    const long long max_by_len = (capacity + 255) / 256;
    if (splits > max_by_len) splits = max_by_len;
    if (splits > 1024) splits = 1024;
    if (splits < 1) splits = 1;
    return (int)splits;
}

hipError_t launch_decode_splitk(const mykfa_decode_params& p, int num_splits, void* ws, hipStream_t stream) {
    DecodeArgs a = make_args(p, num_splits, ws);
    if (p.fwd.dtype == MYKFA_BF16) return splitk_dtype<BF16>(a, p.fwd.head_dim, p.fwd.num_kv_heads, stream);
    return splitk_dtype<FP16>(a, p.fwd.head_dim, p.fwd.num_kv_heads, stream);
}

hipError_t launch_decode_merge(const mykfa_decode_params& p, int num_splits, const void* ws, hipStream_t stream) {
    if (num_splits <= 1) return hipSuccess;
    DecodeArgs a = make_args(p, num_splits, const_cast<void*>(ws));
    if (p.fwd.dtype == MYKFA_BF16) return merge_dtype<BF16>(a, p.fwd.head_dim, stream);
    return merge_dtype<FP16>(a, p.fwd.head_dim, stream);
}

hipError_t launch_kv_append(const mykfa_kv_append_params& p, hipStream_t stream) {
    const long long total = (long long)p.batch * p.seqlen_new * p.num_kv_heads * (p.head_dim / 8);
    long long blocks = (total + 255) / 256;
    if (blocks > 65535) blocks = 65535;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace mykfa
