// Backward pass (replaces _bwd_dq_kernel and _bwd_dkdv_kernel, flash_attn.py:157-314). No
// result is accumulated with atomics: results are bitwise deterministic. (The only atomics are
// the block-queue counters of the queued stored-dS dK/dV kernel, which decide which workgroup
// takes a block, never what it computes.) Two schedules over the same kernels:
//
// Recomputing (mykfa_bwd; every head_dim): two launches in stream order.
//   1. dQ: forward-shaped: delta = rowsum(dO * O) for the workgroup's rows first (the
//      preprocess fused into _bwd_dq_kernel, flash_attn.py:215-216), written for pass 2; then
//      S^T = K Q^T, dP^T = V dO^T, dS^T = P^T (dP^T - delta), and dQ^T += K^T dS^T with K^T read
//      transposed from the LDS K tile.
//   2. dK/dV: one workgroup per 32-key block of one KV head (4 waves = up to 4 query heads of
//      the GQA group); K and V stay in registers as MFMA B operands while each wave streams
//      the query tiles of its head through a wave-private LDS ring, so K/V are read once per
//      group (flash_attn.py:300-311). Per 32-query step a wave computes S = Q K^T and
//      dP = dO V^T (A operands: row reads of the LDS Q/dO tiles), P = exp2(S * c - lse),
//      dS = P (dP - delta), then dV^T += dO^T P and dK^T += Q^T dS with dO^T / Q^T taken by the
//      LDS transpose read.
//
// Stored dS (mykfa_bwd_ws; head_dim 128): delta by bwd_delta_kernel, then per pass of KV heads
// the dK/dV kernel above, which also stores each 32 x 32 block of dS (bf16, the value its dK
// product uses) into a caller's workspace, and bwd_dq_ds_kernel, which forms dQ = dS K from
// those blocks: five products per (query tile, key block) pair instead of seven, paid for
// with one write and one read of dS through HBM.
//
// bwd_delta_kernel alone is mykfa_bwd_preprocess, for callers that run dK/dV without dQ. All
// products are 32x32x16 bf16 (or fp16) MFMA with fp32 accumulation; P and dS are rounded to
// the input type before their products, as in flash_attn.py:177, :257, :260.
#include "common.h"
#include "kernels.h"

namespace mykfa {

namespace {

struct BwdArgs {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const uint16_t* o;
    const uint16_t* dout;
    uint16_t* dq;
    uint16_t* dk;
    uint16_t* dv;
    const float* lse;
    float* delta;
    int64_t qbs, qts, qhs, kbs, kts, khs, vbs, vts, vhs, obs, ots, ohs;
    int64_t dobs, dots, dohs, dqbs, dqts, dqhs, dkbs, dkts, dkhs, dvbs, dvts, dvhs;
    int64_t lse_hs;
    const int32_t* cu_q;
    const int32_t* cu_k;
    int seqlen_q, seqlen_k;
    int wl, wr;
    float qk_scale;
    float sm_scale;
    int group;
    int hpw;
    int num_heads;
    int batch;
    int gx, gy, gz;  // blocks per (group, sequence), sequences, groups; decoded by block_coord
    // Stored dS (the dK/dV pass writes it, the dS-driven dQ pass reads it). A pass covers the
    // query heads of KV heads kv0, kv0 + 1, ...; its r-th query head's blocks start at
    // ds + r * ds_hs (ds_blocks 2 KB blocks each); there, sequence b's rows start at block
    // ds_seq_base(b) (compact rows, see ds_row_off).
    uint16_t* ds;
    int64_t ds_hs;
    int64_t ds_blocks;
    const int64_t* ds_base;  // packed batches: first block of each sequence (device table)
    int64_t ds_seq_dense;    // dense batches: blocks per sequence
    int kv0;
    // Block queues of the queued (persistent) stored-dS dK/dV kernel: kQueueSet ints per pass
    // (one counter per XCD queue) at sched + pass * kQueueSet; the delta kernel zeroes
    // sched_zero of them. sched == nullptr: grid launch.
    int* sched;
    int sched_zero;
};

typedef __attribute__((address_space(1))) s16x8 gs16x8;

// First 32-key block a 32-row query tile i sees (the tile's band starts at key 32 i + lo_f).
__device__ inline int ds_first_block(int i, int lo_f) { return max(i + (lo_f >> 5), 0); }

// ---- compact stored-dS rows ------------------------------------------------------------
//
// Query tile i of a sequence owns one row of 2 KB dS blocks, slot = key block - the first key
// block it sees, with exactly as many slots as its band touches: the first block is
// clamp(i + c_lo, 0, N) and the end clamp(i + c_hi, 0, N) for a full tile, with
// c_lo = floor(lo_f / 32), c_hi = 1 + ceil(hi_f / 32) and N the sequence's key blocks
// (the last, partial tile touches no more). Row i therefore starts at
//   row_off(i) = sum_{i' < i} clamp(i' + c_hi, 0, N) - sum_{i' < i} clamp(i' + c_lo, 0, N),
// each sum in closed form, so the dK/dV writer and the dQ reader locate any row without a
// table; a sequence's rows take row_off(tiles) blocks (a causal sequence of n tiles:
// n (n + 1) / 2, where rows of the longest sequence's width took n * n_max). Sequences follow
// one another: dense batch b at b * blocks(seqlen_q, seqlen_k); packed sequences at the
// prefix sums of their own sizes, a table built on the device before the dK/dV pass
// (ds_build_table). Query heads outermost.
struct DsBand {
    int c_lo, c_hi, nkb;
};
__host__ __device__ inline DsBand ds_band(int q_len, int k_len, int wl, int wr) {
    const int lo_f = band_lo(k_len, q_len, wl), hi_f = band_hi(k_len, q_len, wr);
    DsBand d;
    d.c_lo = lo_f >> 5;               // floor(lo_f / 32)
    d.c_hi = 1 - ((-hi_f) >> 5);      // 1 + ceil(hi_f / 32)
    d.nkb = (k_len + 31) >> 5;
    return d;
}
// sum_{i' < i} clamp(i' + c, 0, n)
__host__ __device__ inline long long ds_clamp_sum(long long c, long long i, long long n) {
    const long long lo = -c < 0 ? 0 : (-c > i ? i : -c);
    const long long hi = n - c < 0 ? 0 : (n - c > i ? i : n - c);
    return (hi - lo) * c + (hi * (hi - 1) - lo * (lo - 1)) / 2 + (i - hi) * n;
}
__host__ __device__ inline long long ds_row_off(const DsBand& d, int i) {
    return ds_clamp_sum(d.c_hi, i, d.nkb) - ds_clamp_sum(d.c_lo, i, d.nkb);
}
// Slots of row i: row_off(i + 1) - row_off(i), for walking consecutive tiles.
__host__ __device__ inline int ds_row_w(const DsBand& d, int i) {
    const int hi = i + d.c_hi < 0 ? 0 : (i + d.c_hi > d.nkb ? d.nkb : i + d.c_hi);
    const int lo = i + d.c_lo < 0 ? 0 : (i + d.c_lo > d.nkb ? d.nkb : i + d.c_lo);
    return hi - lo;
}
__host__ __device__ inline long long ds_seq_blocks(int q_len, int k_len, int wl, int wr) {
    if (q_len <= 0 || k_len <= 0) return 0;
    return ds_row_off(ds_band(q_len, k_len, wl, wr), (q_len + 31) >> 5);
}
// First block of sequence b's rows within a query head's dS.
__device__ inline int64_t ds_seq_base(const BwdArgs& a, int b) {
    return a.cu_q != nullptr ? a.ds_base[b] : (int64_t)b * a.ds_seq_dense;
}

// The packed batch's table of sequence starts (exclusive prefix sums of ds_seq_blocks over the
// sequences, ds_base[batch] = the total), by one block of NT threads: each thread sums a run of
// consecutive sequences (eight length reads in flight at a time), then one block-wide scan
// over the runs. Must complete before the dK/dV pass that stores dS (stream order).
template <int NT>
__device__ void ds_build_table(const BwdArgs& a, int64_t* table) {
    __shared__ int64_t part[NT / 64];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int per = (a.batch + NT - 1) / NT;
    const int b0 = tid * per, b1 = min(b0 + per, a.batch);
    auto blocks = [&](int b) {
        const int ql = a.cu_q[b + 1] - a.cu_q[b], kl = a.cu_k[b + 1] - a.cu_k[b];
        return ds_seq_blocks(ql, kl, a.wl, a.wr);
    };
    int64_t run = 0;
    for (int b = b0; b < b1; b += 8) {
        int64_t s[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) s[u] = b + u < b1 ? blocks(b + u) : 0;
#pragma unroll
        for (int u = 0; u < 8; ++u) run += s[u];
    }
    // Block-wide exclusive scan of the runs.
    int64_t inc = run;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int64_t y = __shfl_up(inc, off);
        if (lane >= off) inc += y;
    }
    if (lane == 63) part[w] = inc;
    __syncthreads();
    int64_t before = 0;
    for (int i = 0; i < w; ++i) before += part[i];
    int64_t at = before + inc - run;
    for (int b = b0; b < b1; b += 8) {
        int64_t s[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) s[u] = b + u < b1 ? blocks(b + u) : 0;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (b + u < b1) table[b + u] = at;
            at += s[u];
        }
    }
    if (b1 == a.batch && b0 < b1) table[a.batch] = at;
    if (a.batch == 0 && tid == 0) table[0] = 0;
}

// Layout of one stored 32 x 32 dS block (bf16, 2 KB): two 1 KB halves by query half
// kb = q / 16; in half kb the 16-byte chunk ds_chunk(kb, g, key) holds queries
// 16 kb + 8 g + 0..7 of key `key`. A dK/dV wave holds exactly these 8 values per lane and
// register group (lane = key + 32 g), so each of its two stores writes 1 KB contiguously
// (16 full cache lines); the XOR places the 16 chunks that one 32-lane transpose read of the
// dQ pass touches (keys r..r+3 x both g x both kb) on distinct banks.
__device__ inline int ds_chunk(int kb, int g, int key) { return 64 * kb + 32 * g + (key ^ (4 * (2 * kb + g))); }

// ---- block queues of the stored-dS dK/dV kernel ------------------------------------------
//
// A grid launch over packed sequences is sized by the longest one: most of its workgroups
// find no work (a rank beyond their sequence) and exit, yet each first waits for a free CU,
// takes its LDS and loads the sequence bounds. On the 17-document 16K-token batch the
// dK/dV grid has 5440 workgroups of which 1064 hold work; the others kept the CUs from the
// long blocks for 11 us at the median and 30 us at worst, and the fixed dispatch order left
// CUs idle for up to 60 us at the end (timestamps per workgroup). The queued kernel runs one
// persistent workgroup per CU instead. Each lists, in LDS, the chunks (kXcdChunk consecutive
// ranks of one (group, sequence) pair, as block_coord numbers them) that hold work, split by
// the XCD the grid launch places them on; it then takes blocks from its own XCD's queue in
// that order (longest first) through one atomic counter per queue, and once that queue is
// empty from the other XCDs' queues. Every block is taken exactly once whatever the
// placement of the workgroups, and a block's outputs depend on nothing else: the results are
// bitwise those of the grid launch. (The dS-driven dQ kernel, run the same way, measured 3%
// slower: its blocks are short and HBM-bound, so the listing and the per-block fetch cost
// more than the idle CUs of its grid launch.)
constexpr int kQueueSet = 8;     // counters per pass: one per XCD queue
constexpr int kQueueCap = 4096;  // chunks a launch may span (LDS list of uint16 entries)
constexpr size_t kSchedBytes = 4096;  // queue counters' share of each KV head's workspace

struct Queues {
    uint16_t list[kQueueCap];  // 16 m + span of each listed chunk c = x + kXcds * m
    int off[kXcds + 1];        // queue x = list[off[x] .. off[x + 1])
    int wsum[16];
    int job;
};

// Lists the chunks c < nchunks that hold work, queue by queue (c % kXcds), each in order, with
// the ranks within the chunk that hold work: span(c, len) = first | last << 2 (0 <= first <=
// last < kXcdChunk), or -1 for none, where len is the length of sequence seq_of(c) (any
// sequence for a padding chunk): cu[seq + 1] - cu[seq], or dense_len without cu. Every read of
// cu goes out before the first is used (unconditionally, at a valid index), so the listing
// costs one memory round trip. NT = threads of the workgroup; the caller guarantees
// nchunks <= kQueueCap.
template <int NT, typename SeqOf, typename Span>
__device__ void build_queues(Queues& qs, int nchunks, SeqOf seq_of, const int32_t* cu, int dense_len, Span span) {
    constexpr int R = (kQueueCap / kXcds + NT - 1) / NT;  // candidates per thread and queue
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    int len[kXcds][R];
#pragma unroll
    for (int x = 0; x < kXcds; ++x)
#pragma unroll
        for (int r = 0; r < R; ++r) len[x][r] = dense_len;
    if (cu != nullptr) {
        int lo[kXcds][R], hi[kXcds][R];
#pragma unroll
        for (int x = 0; x < kXcds; ++x)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int sq = seq_of(x + kXcds * (tid + r * NT));
                lo[x][r] = cu[sq];
                hi[x][r] = cu[sq + 1];
            }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int x = 0; x < kXcds; ++x)
#pragma unroll
            for (int r = 0; r < R; ++r) len[x][r] = hi[x][r] - lo[x][r];
    }
    int base = 0;
#pragma unroll
    for (int x = 0; x < kXcds; ++x) {
        if (tid == 0) qs.off[x] = base;
        const int M = nchunks > x ? (nchunks - x + kXcds - 1) / kXcds : 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (r * NT >= M) break;
            const int m = tid + r * NT;
            const int f = m < M ? span(x + kXcds * m, len[x][r]) : -1;
            const bool v = f >= 0;
            const uint64_t bal = __ballot(v);
            if (lane == 0) qs.wsum[w] = __popcll(bal);
            __syncthreads();
            int before = base, tot = 0;
            for (int i = 0; i < NT / 64; ++i) {
                before += i < w ? qs.wsum[i] : 0;
                tot += qs.wsum[i];
            }
            if (v) qs.list[before + __popcll(bal & ((1ull << lane) - 1))] = (uint16_t)(16 * m + f);
            base += tot;
            __syncthreads();
        }
    }
    if (tid == 0) qs.off[kXcds] = base;
    __syncthreads();
}

// The next block for this workgroup (logical index, as block_coord takes it), or -1 once
// every queue is empty. q (thread 0's copy) is the queue offset from the workgroup's own XCD
// it currently draws from; it only moves on. Ranks of a chunk outside its span are passed over
// without a barrier. Block-uniform call.
__device__ int next_block(Queues& qs, int* ctr, int xcd, int& q) {
    if (threadIdx.x == 0) {
        int job = -1;
        while (q < kXcds) {
            const int x = (xcd + q) & (kXcds - 1);
            const int n = (qs.off[x + 1] - qs.off[x]) * kXcdChunk;
            const int k = n > 0 ? __hip_atomic_fetch_add(ctr + x, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : n;
            if (k >= n) {
                ++q;
                continue;
            }
            const int e = qs.list[qs.off[x] + k / kXcdChunk], lo = k % kXcdChunk;
            if (lo < (e & 3) || lo > ((e >> 2) & 3)) continue;
            job = (x + kXcds * (e >> 4)) * kXcdChunk + lo;
            break;
        }
        qs.job = job;
    }
    __syncthreads();
    const int job = qs.job;
    __syncthreads();
    return job;
}

// Span code (see build_queues) of the chunk whose ranks start at r0 when ranks [lo, hi) of
// its pair hold work; -1 for none.
__device__ inline int rank_span(int r0, int lo, int hi, bool pair_ok) {
    const int f = lo > r0 ? lo - r0 : 0, l = (hi < r0 + kXcdChunk ? hi : r0 + kXcdChunk) - 1 - r0;
    return pair_ok && f <= l ? f | l << 2 : -1;
}

// The kernel's argument block, read afresh by each block of a queued kernel: without the
// opaque pointer the compiler hoists every argument load out of the block loop and keeps the
// values in SGPRs across all of a block's work (114 SGPR and 10 VGPR spills in the dK/dV
// kernel). The argument is the kernel's only one, at offset 0 of the argument segment.
__device__ inline const BwdArgs& fresh_args() {
    auto kp = __builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(kp));
    return *(const BwdArgs*)kp;
}

// The two stored-dS halves' set-up, one block of 64 threads: the block-queue counters start at
// zero, and packed batches get their sequence-start table.
__global__ __launch_bounds__(64) void sched_zero_kernel(BwdArgs a) {
    for (int i = threadIdx.x; i < a.sched_zero; i += blockDim.x) a.sched[i] = 0;
    if (a.ds_base != nullptr) ds_build_table<64>(a, const_cast<int64_t*>(a.ds_base));
}

// ---- 1. delta = rowsum(dO * O) ---------------------------------------------------------

// One flat grid over the (row, head) items: rows run over the packed tokens (varlen:
// cu_seqlens_q[0] .. cu_seqlens_q[batch]) or batch x seqlen_q (dense), heads fastest, D / 8
// lanes per item; each lane keeps U items' loads in flight and the grid strides over the
// rest (a per-sequence grid sized by max_seqlen left most workgroups idle on packed batches:
// 41 -> 28 us at 16384 packed tokens, 16 heads, D = 128).
template <int D, typename T>
__global__ __launch_bounds__(256) void bwd_delta_kernel(BwdArgs a) {
    constexpr int CPR = D / 8;
    constexpr int IPB = 256 / CPR;  // items per block per pass
    constexpr int U = 4;
    const bool varlen = a.cu_q != nullptr;
    const int r_lo = varlen ? a.cu_q[0] : 0;
    const int r_hi = varlen ? a.cu_q[a.batch] : a.batch * a.seqlen_q;
    const int64_t n = (int64_t)(r_hi - r_lo) * a.num_heads;
    // The queue counters of the passes that follow start at zero; packed batches get their
    // dS sequence-start table (by the last block, which has the fewest items).
    if (a.sched != nullptr && blockIdx.x == 0)
        for (int i = threadIdx.x; i < a.sched_zero; i += 256) a.sched[i] = 0;
    if (a.ds_base != nullptr && blockIdx.x == gridDim.x - 1) ds_build_table<256>(a, const_cast<int64_t*>(a.ds_base));
    const int ch = threadIdx.x % CPR;
    const int64_t stride = (int64_t)gridDim.x * IPB;
    for (int64_t base = (int64_t)blockIdx.x * IPB + threadIdx.x / CPR; base < n; base += stride * U) {
        s16x8 ov[U], dv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t item = base + u * stride;
            ov[u] = dv[u] = s16x8{0, 0, 0, 0, 0, 0, 0, 0};
            if (item < n) {
                const int r = r_lo + (int)(item / a.num_heads), h = (int)(item % a.num_heads);
                const int bi = varlen ? 0 : r / a.seqlen_q, t = varlen ? r : r % a.seqlen_q;
                ov[u] = ld16(a.o + (int64_t)bi * a.obs + (int64_t)t * a.ots + (int64_t)h * a.ohs + ch * 8);
                dv[u] = ld16(a.dout + (int64_t)bi * a.dobs + (int64_t)t * a.dots + (int64_t)h * a.dohs + ch * 8);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float sum = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) sum += T::to_float((uint16_t)ov[u][i]) * T::to_float((uint16_t)dv[u][i]);
#pragma unroll
            for (int off = 1; off < CPR; off <<= 1) sum += __shfl_xor(sum, off);
            const int64_t item = base + u * stride;
            if (item < n && ch == 0) {
                const int r = r_lo + (int)(item / a.num_heads), h = (int)(item % a.num_heads);
                a.delta[(int64_t)h * a.lse_hs + r] = sum;
            }
        }
    }
}

// ---- 2. dK / dV -------------------------------------------------------------------------

// A operand (32 rows x 16 k) of a row-major LDS tile at rows perm32(l32), k-step kk.
template <int D>
__device__ inline s16x8 lds_row_op(const uint16_t* tile, int rbase, int l32, int g, int kk) {
    const int row = rbase + perm32(l32);
    return *reinterpret_cast<const s16x8*>(tile + row * D + (((2 * kk + g) ^ lds_swz<D>(row)) << 3));
}

// A operand (32 columns d x 16 rows) of the transposed LDS tile: lane holds
// tile[16 kb + 8 g + i][32 db + l32], through two transpose reads. Columns beyond D read 0.
template <int D>
__device__ inline s16x8 lds_tr_op(const uint16_t* tile, int db, int kb, int lane) {
    const int G = lane >> 4, jj = lane & 15;
    int col = 32 * db + 16 * (G & 1) + 4 * (jj & 3);
    const bool valid = col < D;
    if (!valid) col = col % D;
    const int row = 16 * kb + 8 * (G >> 1) + (jj >> 2);
    s16x8 v = cat4(ds_read_tr(tile + lds_off<D>(row, col)), ds_read_tr(tile + lds_off<D>(row + 4, col)));
    if (!valid) v = s16x8{0, 0, 0, 0, 0, 0, 0, 0};
    return v;
}

// One workgroup = NW waves over one KV head: hpw = gcd(group, NW) waves share each 32-key
// block, each streaming a different query head of the group (heads hs, hs + hpw, ...), so a
// key block's serial chain is group / hpw heads long instead of group. Each wave keeps its
// keys' K and V in registers as B operands and streams its own (Q, dO, lse, delta) query
// tiles through a wave-private asynchronous LDS ring: the main loop has no workgroup
// barrier. The hpw partial dK/dV of a key block are summed through LDS in a fixed order
// (deterministic) at the end. With DS, every 32 x 32 dS block is also stored (bf16, the
// rounding its dV/dK product uses) for the dS-driven dQ pass, in the ds_chunk layout.
template <int D, int NW, int STAGES, typename T, bool DS>
__global__ __launch_bounds__(NW * 64) void bwd_dkdv_kernel(BwdArgs a) {
    constexpr int KD = D / 16;
    constexpr int DB = (D + 31) / 32;
    constexpr int BMQ = 32;
    constexpr int CPR = D / 8;
    constexpr int QLOADS = BMQ * CPR / 64;          // 64-lane loads per 32 x D tile
    constexpr int LOADS = 2 * QLOADS + 2;           // Q, dO, lse, delta
    constexpr int TILE = BMQ * D;                   // elements of one 32 x D tile
    constexpr int STAGE = 2 * TILE + 2 * BMQ * 2;   // Q, dO and 64 floats, in 16-bit units
    static_assert(QLOADS >= 1, "tile must be whole 64-lane loads");
    static_assert(NW * STAGES * STAGE >= NW * DB * 16 * 64 * 2, "reduction buffer fits the ring");
    __shared__ __attribute__((aligned(16))) uint16_t smem[NW][STAGES][STAGE];

    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int l32 = lane & 31, g = lane >> 5;
    const int hpw = a.hpw, kpw = NW / hpw;
    const int kb_w = wave / hpw, hs = wave % hpw;
    // Key blocks are ranked from the END of each sequence: under a causal mask key block n of
    // a sequence of nblk blocks sees nblk - n query blocks, so equal ranks carry equal work in
    // every sequence and rank 0 (the first key block of the longest sequences) starts first.
    const BlockCoord bc = block_coord(xcd_logical(blockIdx.x), a.gz, a.gy, a.cu_k != nullptr);
    if (bc.rank >= a.gx) return;
    const int kvh = a.kv0 + bc.group;
    const int b = bc.seq;
    SeqInfo ks = seq_info(b, a.cu_k, nullptr, a.seqlen_k, false);
    const int k_len = ks.len;
    const int kblk = bc.rank - (a.gx - (k_len + 32 * kpw - 1) / (32 * kpw));
    if (kblk < 0) return;
    const int n0 = kblk * 32 * kpw;
    SeqInfo qs = seq_info(b, a.cu_q, nullptr, a.seqlen_q, false);
    const int q_len = qs.len;
    // Query i sees key j iff (i - j) in [q_len - k_len - wr, q_len - k_len + wl]
    // (flash_attn.py:294-296); forward-oriented offsets for the element mask.
    const int lo_t = band_lo(q_len, k_len, a.wr), hi_t = band_hi(q_len, k_len, a.wl);
    const int lo_f = band_lo(k_len, q_len, a.wl), hi_f = band_hi(k_len, q_len, a.wr);

    const int nw0 = n0 + 32 * kb_w;
    const int bs = k_len - nw0 < 32 ? k_len - nw0 : 32;
    Ranges wr = {0, 0, 0, 0};
    if (bs > 0) wr = block_ranges(nw0, bs, lo_t, hi_t, q_len, BMQ);
    const int ntiles = (bs > 0 && wr.hi > wr.lo) ? (wr.hi - wr.lo + BMQ - 1) / BMQ : 0;
    const int iters = ntiles * (a.group / hpw);

    // K, V rows of this wave as B operands: lane holds K[nw0 + l32][16 kk + 8 g + i]. At
    // D <= 128 they are loaded after the ring's first tiles are issued, so the two latencies
    // overlap, and awaited (with those tiles) before the loop: the compiler places its own
    // wait for a load issued before a loop at the load's first use inside it, where that
    // wait would run every iteration and drain the ring's prefetched tile each time. (At
    // D = 256 the compiler crashes on that order; there they load first and land before the
    // ring.)
    s16x8 kop[KD], vop[KD];
    auto load_kv = [&]() {
        const int key = nw0 + l32;
        const uint16_t* kp = a.k + (int64_t)b * a.kbs + (ks.tok0 + key) * a.kts + (int64_t)kvh * a.khs;
        const uint16_t* vp = a.v + (int64_t)b * a.vbs + (ks.tok0 + key) * a.vts + (int64_t)kvh * a.vhs;
#pragma unroll
        for (int kk = 0; kk < KD; ++kk) {
            s16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
            kop[kk] = key < k_len ? ld16(kp + 16 * kk + 8 * g) : z;
            vop[kk] = key < k_len ? ld16(vp + 16 * kk + 8 * g) : z;
        }
    };
    if constexpr (D > 128) {
        load_kv();
        wait_vmcnt<0>();  // K/V landed before the ring's loads share the counter
    }
    // Output rows of this lane's key, formed here so that no kernel argument stays live
    // across the main loop (they would be spilled from scalar registers).
    const int out_key = nw0 + l32;
    uint16_t* const dkp = a.dk + (int64_t)b * a.dkbs + (ks.tok0 + out_key) * a.dkts + (int64_t)kvh * a.dkhs;
    uint16_t* const dvp = a.dv + (int64_t)b * a.dvbs + (ks.tok0 + out_key) * a.dvts + (int64_t)kvh * a.dvhs;
    const float sm_scale = a.sm_scale, qk_scale = sgpr_copy(a.qk_scale);
    const int64_t q_hstep = (int64_t)hpw * a.qhs, do_hstep = (int64_t)hpw * a.dohs;
    const int64_t f_hstep = (int64_t)hpw * a.lse_hs, qts = sgpr_copy(a.qts), dots = sgpr_copy(a.dots);
    f32x16 dk[DB], dv[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) dk[db][r] = dv[db][r] = 0.f;

    uint16_t* ring = smem[wave][0];
    const uint32_t ring_lds = lds_addr(ring);
    // Iteration it streams query tile it % ntiles of head hs + hpw * (it / ntiles). The issue
    // side keeps its own (tile, head) state: stream pointers of its current head, advanced by
    // hpw heads after ntiles tiles, so the loop does no division and little 64-bit math.
    const int h0 = kvh * a.group + hs;
    const uint16_t* iq = a.q + (int64_t)b * a.qbs + qs.tok0 * a.qts + (int64_t)h0 * a.qhs;
    const uint16_t* ido = a.dout + (int64_t)b * a.dobs + qs.tok0 * a.dots + (int64_t)h0 * a.dohs;
    const float* ilse = a.lse + (int64_t)h0 * a.lse_hs + qs.row0;
    const float* idel = a.delta + (int64_t)h0 * a.lse_hs + qs.row0;  // lse's (head, row) layout
    // Lane offsets inside a 32-row tile (row-relative, swizzled 16-byte chunk): the tile's
    // first row goes into the buffer base, so these are loop-invariant.
    unsigned q_lane[QLOADS], do_lane[QLOADS];
#pragma unroll
    for (int j = 0; j < QLOADS; ++j) {
        const int p = j * 64 + lane;
        const int row = p / CPR, logical = (p % CPR) ^ lds_swz<D>(row);
        q_lane[j] = (unsigned)(row * (int)(a.qts * 2) + logical * 16);
        do_lane[j] = (unsigned)(row * (int)(a.dots * 2) + logical * 16);
    }
    const unsigned f_lane = (unsigned)((lane & 31) * 4);
    // Issue-side state, advanced by additions only: the addresses of the next tile's first Q,
    // dO and lse rows, and the bytes from each to the end of the sequence's rows (the
    // descriptors' ranges: rows at or beyond q_len read 0). After ntiles tiles they move to the
    // next head of the wave (hpw heads on). delta shares lse's (head, row) layout, so its
    // address is lse's plus a fixed distance.
    const uint64_t q_tstep = (uint64_t)(BMQ * qts) * 2, do_tstep = (uint64_t)(BMQ * dots) * 2;
    const int rows0 = q_len - wr.lo;  // >= 1 whenever a tile is issued
    const int qb0 = rows0 > 0 ? (int)(((int64_t)(rows0 - 1) * qts + D) * 2) : 0;
    const int dob0 = rows0 > 0 ? (int)(((int64_t)(rows0 - 1) * dots + D) * 2) : 0;
    const int fb0 = rows0 * 4;
    uint64_t hq = reinterpret_cast<uint64_t>(iq + (int64_t)wr.lo * qts);
    uint64_t hdo = reinterpret_cast<uint64_t>(ido + (int64_t)wr.lo * dots);
    uint64_t hf = reinterpret_cast<uint64_t>(ilse + wr.lo);
    const uint64_t dl = reinterpret_cast<uint64_t>(idel) - reinterpret_cast<uint64_t>(ilse);
    const uint64_t q_hb = (uint64_t)q_hstep * 2, do_hb = (uint64_t)do_hstep * 2, f_hb = (uint64_t)f_hstep * 4;
    uint64_t tq = hq, tdo = hdo, tf = hf;
    int qb = qb0, dob = dob0, fb = fb0;
    int iss_tile = 0, iss_stage = 0;
    auto issue = [&]() {
        const uint32_t st = ring_lds + iss_stage * (STAGE * 2);
        const uint32_t fl = st + 2 * TILE * 2;  // lse into floats [0, 32), delta into [32, 64)
        if constexpr (D <= 128) {
            const i32x4 rq = buffer_rsrc32(tq, qb);
            const i32x4 rd = buffer_rsrc32(tdo, dob);
#pragma unroll
            for (int j = 0; j < QLOADS; ++j) {
                dma16(rq, st + j * 1024, q_lane[j]);
                dma16(rd, st + (TILE + j * 512) * 2, do_lane[j]);
            }
            if (lane < 32) dma4(buffer_rsrc32(tf, fb), fl, f_lane);
            if (lane >= 32) dma4(buffer_rsrc32(tf + dl, fb), fl, f_lane);
        } else {
            // Same tiles from the head pointers (the compiler's AGPR rewrite pass crashes on
            // the incremental form at D = 256).
            const int m0 = wr.lo + iss_tile * BMQ;
            const i32x4 rq = rows_rsrc(iq + m0 * qts, q_len - m0, qts, D);
            const i32x4 rd = rows_rsrc(ido + m0 * dots, q_len - m0, dots, D);
#pragma unroll
            for (int j = 0; j < QLOADS; ++j) {
                dma16(rq, st + j * 1024, q_lane[j]);
                dma16(rd, st + (TILE + j * 512) * 2, do_lane[j]);
            }
            const int64_t fbytes = (int64_t)(q_len - m0) * 4;
            if (lane < 32) dma4(buffer_rsrc(ilse + m0, fbytes), fl, f_lane);
            if (lane >= 32) dma4(buffer_rsrc(idel + m0, fbytes), fl, f_lane);
        }
        iss_stage = iss_stage + 1 == STAGES ? 0 : iss_stage + 1;
        if (++iss_tile == ntiles) {
            iss_tile = 0;
            if constexpr (D <= 128) {
                hq += q_hb;
                hdo += do_hb;
                hf += f_hb;
                tq = hq;
                tdo = hdo;
                tf = hf;
                qb = qb0;
                dob = dob0;
                fb = fb0;
            } else {
                iq += q_hstep;
                ido += do_hstep;
                ilse += f_hstep;
                idel += f_hstep;
            }
        } else if constexpr (D <= 128) {
            tq += q_tstep;
            tdo += do_tstep;
            tf += BMQ * 4;
            qb -= (int)q_tstep;
            dob -= (int)do_tstep;
            fb -= BMQ * 4;
        }
    };
    // Every stage is filled up front, and a stage is refilled (tile it + STAGES) as soon as
    // iteration it has read it, before that iteration's dV/dK products: a tile gets about
    // STAGES - 1/2 iterations to land rather than STAGES - 1.
#pragma unroll
    for (int t = 0; t < STAGES; ++t)
        if (t < iters) issue();
    if constexpr (D <= 128) {
        load_kv();
        wait_vmcnt<0>();
    }

    // dS: byte address of the current head's (pass-relative) first row of this sequence, moved
    // on by hpw heads per head change; the lane's 16-byte chunk within a block.
    uint64_t ds_ptr = 0, ds_hstep = 0;
    int ds_jblk = 0, ds_lob = 0;
    int64_t ds_room = 0;  // blocks of the head's dS from this sequence's first row on
    DsBand ds_bd = {0, 0, 0};
    if constexpr (DS) {
        const int64_t base = ds_seq_base(a, b);
        ds_room = a.ds_blocks - base;
        ds_bd = ds_band(q_len, k_len, a.wl, a.wr);
        ds_hstep = (uint64_t)hpw * (uint64_t)a.ds_hs * 2;
        ds_ptr = reinterpret_cast<uint64_t>(a.ds) +
                 ((uint64_t)((int64_t)(kvh - a.kv0) * a.group + hs) * (uint64_t)a.ds_hs + (uint64_t)base * 1024) * 2;
        ds_jblk = nw0 >> 5;
        ds_lob = lo_f >> 5;
    }
    const unsigned ds_lane0 = (unsigned)(ds_chunk(0, g, l32) * 16), ds_lane1 = (unsigned)(ds_chunk(1, g, l32) * 16);
    const bool partial_block = bs < 32;
    // A tile's dS block is stored at the top of the NEXT iteration, right after its ring wait:
    // stores share the vector memory counter with the ring loads, and a store issued before
    // a refill would hold up the wait for the tile after it until the store completed.
    s16x8 ds_keep[2] = {s16x8{0, 0, 0, 0, 0, 0, 0, 0}, s16x8{0, 0, 0, 0, 0, 0, 0, 0}};
    uint64_t ds_keep_at = 0;
    bool ds_keep_ok = false;
    auto ds_flush = [&]() {
        if (ds_keep_ok) {
            // Global (not generic) address space: a flat store would also count against the
            // LDS counter and hold up every LDS wait until it completed.
            *reinterpret_cast<gs16x8*>(ds_keep_at + ds_lane0) = ds_keep[0];
            *reinterpret_cast<gs16x8*>(ds_keep_at + ds_lane1) = ds_keep[1];
        }
        ds_keep_ok = false;
    };

    int cur_tile = 0, cur_stage = 0;
    for (int it = 0; it < iters; ++it) {
        const int after = iters - 1 - it < STAGES - 1 ? iters - 1 - it : STAGES - 1;
        ring_wait<LOADS, STAGES + 1>(after);  // tile it landed; up to STAGES - 1 later tiles in flight
        if constexpr (DS) ds_flush();
        const int m0 = wr.lo + cur_tile * BMQ;
        const bool masked = !(m0 >= wr.mid_lo && m0 + BMQ <= wr.mid_hi);
        const uint16_t* st = ring + cur_stage * STAGE;
        const bool head_done = cur_tile + 1 == ntiles;
        cur_tile = cur_tile + 1 == ntiles ? 0 : cur_tile + 1;
        cur_stage = cur_stage + 1 == STAGES ? 0 : cur_stage + 1;
        const uint16_t* Qs = st;
        const uint16_t* DOs = st + TILE;
        const float* fl = reinterpret_cast<const float*>(st + 2 * TILE);
        // S = Q K^T and dP = dO V^T: lane column = key nw0 + l32, registers = queries.
        f32x16 s, dp;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
#pragma unroll
        for (int kk = 0; kk < KD; ++kk) {
            s = T::mfma32(lds_row_op<D>(Qs, 0, l32, g, kk), kop[kk], s);
            dp = T::mfma32(lds_row_op<D>(DOs, 0, l32, g, kk), vop[kk], dp);
        }
        // Transposed operands of dV/dK, read now so their latency hides under the VALU work
        // (D <= 128; at D = 256 the registers are not there).
        constexpr bool PF = D <= 128;
        s16x8 dot_op[PF ? DB : 1][2], qt_op[PF ? DB : 1][2];
        if constexpr (PF) {
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    dot_op[db][kb] = lds_tr_op<D>(DOs, db, kb, lane);
                    qt_op[db][kb] = lds_tr_op<D>(Qs, db, kb, lane);
                }
            __builtin_amdgcn_sched_barrier(0);
        }
        const int key = nw0 + l32;
        // Register r = 8 kb + i holds query row m0 + 16 kb + 8 g + i; its lse / delta sit at
        // floats [16 kb + 8 g + i] / [32 + 16 kb + 8 g + i] of the stage.
        float pv[16], lsev[16], delv[16];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const f32x4 l0 = *reinterpret_cast<const f32x4*>(fl + 16 * kb + 8 * g);
            const f32x4 l1 = *reinterpret_cast<const f32x4*>(fl + 16 * kb + 8 * g + 4);
            const f32x4 d0 = *reinterpret_cast<const f32x4*>(fl + 32 + 16 * kb + 8 * g);
            const f32x4 d1 = *reinterpret_cast<const f32x4*>(fl + 32 + 16 * kb + 8 * g + 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                lsev[8 * kb + i] = l0[i];
                lsev[8 * kb + 4 + i] = l1[i];
                delv[8 * kb + i] = d0[i];
                delv[8 * kb + 4 + i] = d1[i];
            }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) pv[r] = fast_exp2(fmaf(s[r], qk_scale, -lsev[r]));
        // Band mask, only on tiles that cross the band edge (flash_attn.py:294-296).
        // Query i is visible from this lane's key iff lo_f <= key - i <= hi_f, i < q_len and
        // key < k_len: one range of query rows (register r = 8 kb + i is row m0 + 16 kb + 8 g + i).
        if (masked) mask_runs16(pv, m0 + 8 * g, key - hi_f, key < k_len ? min(key - lo_f, q_len - 1) : key - hi_f - 1);
        s16x8 pb[2], dsb[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            float dsv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) dsv[i] = pv[8 * kb + i] * (dp[8 * kb + i] - delv[8 * kb + i]);
            const float* pk = pv + 8 * kb;
            u32x4 pw = {T::pack2(pk[0], pk[1]), T::pack2(pk[2], pk[3]), T::pack2(pk[4], pk[5]), T::pack2(pk[6], pk[7])};
            u32x4 dw = {T::pack2(dsv[0], dsv[1]), T::pack2(dsv[2], dsv[3]), T::pack2(dsv[4], dsv[5]),
                        T::pack2(dsv[6], dsv[7])};
            pb[kb] = __builtin_bit_cast(s16x8, pw);
            dsb[kb] = __builtin_bit_cast(s16x8, dw);
        }
        if constexpr (DS) {
            // Block (tile m0 / 32, key block nw0 / 32): lane (key l32, g) holds queries
            // 16 kb + 8 g + 0..7 of its key. Keys past the sequence are stored as 0 (their K
            // rows are 0 and their scores unmasked inside the band's full tiles).
            const int ti = m0 >> 5;
            const int slot = ds_jblk - max(ti + ds_lob, 0);  // ds_first_block(ti, lo_f)
            ds_keep[0] = dsb[0];
            ds_keep[1] = dsb[1];
            if (partial_block && key >= k_len) ds_keep[0] = ds_keep[1] = s16x8{0, 0, 0, 0, 0, 0, 0, 0};
            const int64_t blk = ds_row_off(ds_bd, ti) + slot;
            ds_keep_ok = slot >= 0 && blk < ds_room;
            ds_keep_at = ds_ptr + (uint64_t)blk * 2048;
            if (head_done) ds_ptr += ds_hstep;
        }
        // With the transposed operands already in registers the stage is free: refill it now
        // (this wave's reads of it have returned), ahead of the dV/dK products.
        if constexpr (PF) {
            wait_lgkmcnt0();
            if (it + STAGES < iters) issue();
        }
        // dV^T += dO^T P, dK^T += Q^T dS.
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                if constexpr (PF) {
                    dv[db] = T::mfma32(dot_op[db][kb], pb[kb], dv[db]);
                    dk[db] = T::mfma32(qt_op[db][kb], dsb[kb], dk[db]);
                } else {
                    dv[db] = T::mfma32(lds_tr_op<D>(DOs, db, kb, lane), pb[kb], dv[db]);
                    dk[db] = T::mfma32(lds_tr_op<D>(Qs, db, kb, lane), dsb[kb], dk[db]);
                }
            }
        if constexpr (!PF) {
            wait_lgkmcnt0();
            if (it + STAGES < iters) issue();
        }
    }
    if constexpr (DS) ds_flush();

    // Sum the hpw partials of each key block in a fixed order (waves hs = 1.. into hs = 0).
    if (hpw > 1) {
        float* red = reinterpret_cast<float*>(&smem[0][0][0]);
        constexpr int PART = DB * 16 * 64;  // floats of one wave's accumulator set
#pragma unroll
        for (int pass = 0; pass < 2; ++pass) {
            f32x16* accs = pass == 0 ? dk : dv;
            __syncthreads();
            if (hs != 0) {
                float* dst = red + wave * PART;
#pragma unroll
                for (int db = 0; db < DB; ++db)
#pragma unroll
                    for (int r = 0; r < 16; ++r) dst[(db * 16 + r) * 64 + lane] = accs[db][r];
            }
            __syncthreads();
            if (hs == 0) {
                for (int o = 1; o < hpw; ++o) {
                    const float* src = red + (wave + o) * PART;
#pragma unroll
                    for (int db = 0; db < DB; ++db)
#pragma unroll
                        for (int r = 0; r < 16; ++r) accs[db][r] += src[(db * 16 + r) * 64 + lane];
                }
            }
        }
    }

    // Store dK * sm_scale and dV (flash_attn.py:312-314); lane column = key, rows = d.
    if (hs == 0 && bs > 0 && out_key < k_len) {
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int rq = 0; rq < 4; ++rq) {
                const int d0 = 32 * db + 8 * rq + 4 * g;
                if (d0 < D) {
                    u32x2 wk = {T::pack2(dk[db][4 * rq] * sm_scale, dk[db][4 * rq + 1] * sm_scale),
                                T::pack2(dk[db][4 * rq + 2] * sm_scale, dk[db][4 * rq + 3] * sm_scale)};
                    u32x2 wv = {T::pack2(dv[db][4 * rq], dv[db][4 * rq + 1]),
                                T::pack2(dv[db][4 * rq + 2], dv[db][4 * rq + 3])};
                    *reinterpret_cast<u32x2*>(dkp + d0) = wk;
                    *reinterpret_cast<u32x2*>(dvp + d0) = wv;
                }
            }
    }
}

// ---- 2b. dK / dV by wave pairs ----------------------------------------------------------
//
// Eight waves = four pairs. The two waves of pair p (waves p and p + 4, which the dispatcher
// places on one SIMD) split a 32-key block's four products between them:
//   wave A (0..3): K and the dV accumulator.  S = Q K^T, P = exp2(S c - lse), dV^T += dO^T P
//   wave B (4..7): V and the dK accumulator.  dP = dO V^T, dS = P (dP - delta), dK^T += Q^T dS
// P crosses from A to B through LDS in fp32, so dS is formed from the same fp32 P as in the
// single-wave kernel above. Each wave holds half of that kernel's resident state (K and dV, or
// V and dK: under 256 registers), so both waves of a pair share one SIMD and one's products run
// while the other computes exponentials or waits for LDS. B works one query tile behind A: in
// step t, A computes S(t), P(t) and dV(t) while B finishes dS(t-1) and dK(t-1) and computes
// dP(t); one workgroup barrier per step publishes P(t) and the next ring tile.
// The four pairs are HPW query heads x KPW = 4 / HPW consecutive 32-key blocks of one KV head.
// The KPW pairs of a head share its (Q, dO, lse, delta) tile ring, streamed over the union of
// their bands (a tile outside one pair's band is fully masked for it), which the A waves of
// those pairs fill between them; every tile is read in the step that consumes it (B keeps its
// transposed Q operands in registers for the next step), so a stage is refilled right after
// the barrier that ends its step and a tile has STAGES - 1 steps to land. The HPW partial
// sums of a key block are added through LDS in a fixed order: no atomics, bitwise repeatable.
// Steps it + S .. it + N - 1 of a loop unrolled by N (those below iters), each called with its
// position S as a compile-time constant.
template <int S, int N, typename F>
__device__ __forceinline__ void stage_steps(F& f, int it, int iters) {
    if constexpr (S < N) {
        if (it + S < iters) {
            f(std::integral_constant<int, S>{}, it + S);
            stage_steps<S + 1, N>(f, it, iters);
        }
    }
}

template <int D, int HPW, int STAGES, typename T, bool DS>
__device__ __forceinline__ void dkdv_pair_block(const BwdArgs& a, int block) {
    constexpr int KPW = 4 / HPW;
    constexpr int KD = D / 16;
    constexpr int DB = D / 32;
    constexpr int BMQ = 32;
    constexpr int CPR = D / 8;
    constexpr int QLOADS = BMQ * CPR / 64;          // 64-lane loads per 32 x D tile
    constexpr int PARTS = KPW / 2;                  // A waves sharing one tensor's loads
    constexpr int TLOADS = QLOADS / PARTS;          // tensor loads per issuing wave and tile
    constexpr int LOADS = TLOADS + 1;               // + the lse or delta row
    constexpr int TILE = BMQ * D;                   // elements of one 32 x D tile
    constexpr int STAGE = 2 * TILE + 2 * BMQ * 2;   // Q, dO and 64 floats, in 16-bit units
    constexpr int XBUF = 16 * 64;                   // floats of one pair's P exchange buffer
    static_assert(HPW == 1 || HPW == 2, "two or four key blocks per workgroup");
    static_assert(QLOADS % PARTS == 0, "tensor loads split evenly over the issuing waves");
    static_assert(HPW == 1 || 2 * STAGES * STAGE * 2 >= 4 * DB * 16 * 64 * 4, "reduction fits the ring");
    __shared__ __attribute__((aligned(16))) uint16_t ring_mem[HPW][STAGES][STAGE];
    __shared__ __attribute__((aligned(16))) float xbuf[STAGES][4][XBUF];

    // The thread index through an opaque copy: in the queued kernel's block loop the compiler
    // would otherwise compute every lane-dependent offset of both roles once before the loop
    // and hold them all across it (10 VGPR spills); the mask restores the known range.
    int tid_raw = threadIdx.x;
    asm volatile("" : "+v"(tid_raw));
    const int tid = tid_raw & 511, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int l32 = lane & 31, g = lane >> 5;
    const bool role_b = wave >= 4;
    const int pair = wave & 3;
    const int hs = pair / KPW, kbi = pair % KPW;
    // Key blocks are ranked from the END of each sequence (see bwd_dkdv_kernel).
    const BlockCoord bc = block_coord(block, a.gz, a.gy, a.cu_k != nullptr);
    if (bc.rank >= a.gx) return;
    const int kvh = a.kv0 + bc.group;
    const int b = bc.seq;
    SeqInfo ks = seq_info(b, a.cu_k, nullptr, a.seqlen_k, false);
    const int k_len = ks.len;
    const int kblk = bc.rank - (a.gx - (k_len + 32 * KPW - 1) / (32 * KPW));
    if (kblk < 0) return;
    const int n0 = kblk * 32 * KPW;
    SeqInfo qs = seq_info(b, a.cu_q, nullptr, a.seqlen_q, false);
    const int q_len = qs.len;
    // Query i sees key j iff (i - j) in [q_len - k_len - wr, q_len - k_len + wl]
    // (flash_attn.py:294-296); forward-oriented offsets for the element mask.
    const int lo_t = band_lo(q_len, k_len, a.wr), hi_t = band_hi(q_len, k_len, a.wl);
    const int lo_f = band_lo(k_len, q_len, a.wl), hi_f = band_hi(k_len, q_len, a.wr);
    // The ring streams the union of the workgroup's bands; each pair masks by its own.
    const int bsu = k_len - n0 < 32 * KPW ? k_len - n0 : 32 * KPW;  // >= 1
    const Ranges ur = block_ranges(n0, bsu, lo_t, hi_t, q_len, BMQ);
    const int ntiles = ur.hi > ur.lo ? (ur.hi - ur.lo + BMQ - 1) / BMQ : 0;
    const int iters = ntiles * (a.group / HPW);
    const int nw0 = n0 + 32 * kbi;
    const int bs = k_len - nw0 < 32 ? k_len - nw0 : 32;
    Ranges wr = {0, 0, 0, 0};
    if (bs > 0) wr = block_ranges(nw0, bs, lo_t, hi_t, q_len, BMQ);
    const int key = nw0 + l32;

    uint16_t* const ring = &ring_mem[hs][0][0];
    const uint32_t ring_lds = lds_addr(ring);
    const int h0 = kvh * a.group + hs;  // first query head of this pair's ring
    f32x16 acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
    // K (wave A) or V (wave B) rows of this pair's keys as B operands: lane holds
    // X[key][16 kk + 8 g + i]; rows past the sequence are 0.
    s16x8 kv[KD];

    if (!role_b) {
        // ---- wave A: ring issue, S, P, dV ----
        // This wave's share of each tile: tensor `tens` (0 = Q, 1 = dO), loads
        // [part * TLOADS, (part + 1) * TLOADS) of it, and the lse (even kbi) or delta row.
        const int tens = kbi / PARTS, part = kbi % PARTS;
        const bool f_delta = (kbi & 1) != 0;
        const int64_t tstride = tens == 0 ? a.qts : a.dots;
        const int64_t thead = tens == 0 ? a.qhs : a.dohs;
        const uint16_t* tbase = tens == 0 ? a.q + (int64_t)b * a.qbs + qs.tok0 * a.qts
                                          : a.dout + (int64_t)b * a.dobs + qs.tok0 * a.dots;
        const float* fbase = (f_delta ? a.delta : a.lse) + qs.row0;
        unsigned t_lane[TLOADS];
#pragma unroll
        for (int j = 0; j < TLOADS; ++j) {
            const int p = (part * TLOADS + j) * 64 + lane;
            const int row = p / CPR, logical = (p % CPR) ^ lds_swz<D>(row);
            t_lane[j] = (unsigned)(row * (int)(tstride * 2) + logical * 16);
        }
        const unsigned f_lane = (unsigned)(lane * 4);
        const uint32_t t_lds = (uint32_t)(tens * TILE * 2 + part * TLOADS * 1024);
        const uint32_t f_lds = (uint32_t)(2 * TILE * 2 + (f_delta ? BMQ * 4 : 0));
        // Issue-side state, advanced by additions: the next tile's first-row address and the
        // bytes from it to the end of the sequence's rows (rows at or beyond q_len read 0);
        // after ntiles tiles both move to the next head of this ring (HPW heads on).
        const int rows0 = q_len - ur.lo;  // >= 1 whenever a tile is issued
        const int tb0 = rows0 > 0 ? (int)(((int64_t)(rows0 - 1) * tstride + D) * 2) : 0;
        const int fb0 = rows0 * 4;
        const uint64_t t_tstep = (uint64_t)(BMQ * tstride) * 2;
        const uint64_t t_hb = (uint64_t)(HPW * thead) * 2, f_hb = (uint64_t)(HPW * a.lse_hs) * 4;
        uint64_t ht = reinterpret_cast<uint64_t>(tbase + (int64_t)h0 * thead + (int64_t)ur.lo * tstride);
        uint64_t hf = reinterpret_cast<uint64_t>(fbase + (int64_t)h0 * a.lse_hs + ur.lo);
        uint64_t tt = ht, tf = hf;
        int tb = tb0, fb = fb0, iss_tile = 0, iss_stage = 0;
        // A tile's loads go out in three chunks spread over the step (loads [J0, J1) of the
        // tensor, then the lse / delta row): issued back to back, the four A waves' loads
        // queue up in the CU's memory pipe and stall their waves for hundreds of cycles.
        auto issue_part = [&](auto J0c, auto J1c, bool with_f) {
            constexpr int J0 = decltype(J0c)::value, J1 = decltype(J1c)::value;
            const uint32_t st = ring_lds + iss_stage * (STAGE * 2);
            const i32x4 rt = buffer_rsrc32(tt, tb);
#pragma unroll
            for (int j = J0; j < J1; ++j) dma16(rt, st + t_lds + j * 1024, t_lane[j]);
            if (with_f && lane < 32) dma4(buffer_rsrc32(tf, fb), st + f_lds, f_lane);
        };
        auto issue_end = [&]() {
            iss_stage = iss_stage + 1 == STAGES ? 0 : iss_stage + 1;
            if (++iss_tile == ntiles) {
                iss_tile = 0;
                ht += t_hb;
                hf += f_hb;
                tt = ht;
                tf = hf;
                tb = tb0;
                fb = fb0;
            } else {
                tt += t_tstep;
                tf += BMQ * 4;
                tb -= (int)t_tstep;
                fb -= BMQ * 4;
            }
        };
        using C0 = std::integral_constant<int, 0>;
        using C1 = std::integral_constant<int, TLOADS / 3>;
        using C2 = std::integral_constant<int, 2 * TLOADS / 3>;
        using C3 = std::integral_constant<int, TLOADS>;
#pragma unroll
        for (int t = 0; t < STAGES - 1; ++t)
            if (t < iters) {
                issue_part(C0{}, C3{}, true);
                issue_end();
            }
        {
            const uint16_t* kp = a.k + (int64_t)b * a.kbs + (ks.tok0 + key) * a.kts + (int64_t)kvh * a.khs;
#pragma unroll
            for (int kk = 0; kk < KD; ++kk) {
                const s16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
                kv[kk] = key < k_len ? ld16(kp + 16 * kk + 8 * g) : z;
            }
        }
        wait_vmcnt<0>();
        barrier_lds();

        const float qk_scale = sgpr_copy(a.qk_scale);
        int cur_tile = 0;
        // One step per query tile; the ring stage (it % STAGES) is a compile-time constant of
        // each unrolled step, so every LDS address of the step is a per-lane register plus an
        // immediate (with a run-time stage the step spent ~40 VALU instructions on addresses).
        auto a_step = [&](auto SC, int it) {
            constexpr int stage = decltype(SC)::value;
            // Tile it + STAGES - 1 goes into the stage tile it - 1 used, in three chunks.
            const bool refill = it + STAGES - 1 < iters;
            if (refill) issue_part(C0{}, C1{}, false);
            const int m0 = ur.lo + cur_tile * BMQ;
            const bool masked = !(m0 >= wr.mid_lo && m0 + BMQ <= wr.mid_hi);
            const uint16_t* Qs = ring + stage * STAGE;
            const uint16_t* DOs = Qs + TILE;
            const float* fl = reinterpret_cast<const float*>(Qs + 2 * TILE);
            cur_tile = cur_tile + 1 == ntiles ? 0 : cur_tile + 1;
            // All operand reads of a product are issued before it (the compiler would otherwise
            // serialize read -> wait -> product): the Q rows and the lse row for S, then the
            // transposed dO operands of dV, whose latency hides under the exponentials.
            s16x8 qa[KD];
#pragma unroll
            for (int kk = 0; kk < KD; ++kk) qa[kk] = lds_row_op<D>(Qs, 0, l32, g, kk);
            f32x4 lq[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) lq[c] = *reinterpret_cast<const f32x4*>(fl + 16 * (c >> 1) + 8 * g + 4 * (c & 1));
            __builtin_amdgcn_sched_barrier(0);
            // S = Q K^T: lane column = key, register r = 8 kb + i holds row m0 + 16 kb + 8 g + i.
            f32x16 s;
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
            for (int kk = 0; kk < KD; ++kk) s = T::mfma32(qa[kk], kv[kk], s);
            s16x8 dot[DB][2];
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) dot[db][kb] = lds_tr_op<D>(DOs, db, kb, lane);
            if (refill) issue_part(C1{}, C2{}, false);
            __builtin_amdgcn_sched_barrier(0);
            float pv[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) pv[r] = fast_exp2(fmaf(s[r], qk_scale, -lq[r >> 2][r & 3]));
            // Band mask on tiles that are not wholly inside this pair's band: query i is
            // visible from this lane's key iff lo_f <= key - i <= hi_f, i < q_len, key < k_len.
            if (masked) mask_runs16(pv, m0 + 8 * g, key - hi_f, key < k_len ? min(key - lo_f, q_len - 1) : key - hi_f - 1);
            // P for wave B, in chunk-major lane order (16-byte writes, conflict-free).
            float* xp = &xbuf[stage][pair][0];
#pragma unroll
            for (int c = 0; c < 4; ++c)
                *reinterpret_cast<f32x4*>(xp + c * 256 + lane * 4) =
                    f32x4{pv[4 * c], pv[4 * c + 1], pv[4 * c + 2], pv[4 * c + 3]};
            s16x8 pb[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const float* pk = pv + 8 * kb;
                u32x4 pw = {T::pack2(pk[0], pk[1]), T::pack2(pk[2], pk[3]), T::pack2(pk[4], pk[5]), T::pack2(pk[6], pk[7])};
                pb[kb] = __builtin_bit_cast(s16x8, pw);
            }
            // dV^T += dO^T P.
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) acc[db] = T::mfma32(dot[db][kb], pb[kb], acc[db]);
            if (refill) {
                issue_part(C2{}, C3{}, true);
                issue_end();
            }
            // Tile it + 1 landed (this wave's loads of it); later tiles may stay in flight.
            const int after = iters - 2 - it < STAGES - 2 ? iters - 2 - it : STAGES - 2;
            if (after >= 0) ring_wait<LOADS, STAGES>(after);
            barrier_lds();
        };
        for (int it = 0; it < iters; it += STAGES) stage_steps<0, STAGES>(a_step, it, iters);
    } else {
        // ---- wave B: dP, dS, dK (one tile behind A) ----
        {
            const uint16_t* vp = a.v + (int64_t)b * a.vbs + (ks.tok0 + key) * a.vts + (int64_t)kvh * a.vhs;
#pragma unroll
            for (int kk = 0; kk < KD; ++kk) {
                const s16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
                kv[kk] = key < k_len ? ld16(vp + 16 * kk + 8 * g) : z;
            }
        }
        wait_vmcnt<0>();
        barrier_lds();

        // dS rows of this pair's first head (pass-relative) in the sequence; moved on by HPW
        // heads per head change.
        uint64_t ds_ptr = 0, ds_hstep = 0;
        int64_t ds_room = 0;  // blocks of the head's dS from this sequence's first row on
        DsBand ds_bd = {0, 0, 0};
        if constexpr (DS) {
            const int64_t base = ds_seq_base(a, b);
            ds_room = a.ds_blocks - base;
            ds_bd = ds_band(q_len, k_len, a.wl, a.wr);
            ds_hstep = (uint64_t)HPW * (uint64_t)a.ds_hs * 2;
            ds_ptr = reinterpret_cast<uint64_t>(a.ds) +
                     ((uint64_t)((int64_t)(kvh - a.kv0) * a.group + hs) * (uint64_t)a.ds_hs + (uint64_t)base * 1024) * 2;
        }
        const int ds_jblk = nw0 >> 5, ds_lob = lo_f >> 5;
        const unsigned ds_lane0 = (unsigned)(ds_chunk(0, g, l32) * 16), ds_lane1 = (unsigned)(ds_chunk(1, g, l32) * 16);
        const bool zero_keys = bs < 32 && key >= k_len;
        // dS(t) = P(t) (dP(t) - delta(t)) and dK^T += Q^T dS for the tile of the previous step,
        // whose dP - delta and transposed Q operands this wave kept in registers.
        f32x16 dpm;
        s16x8 qt[DB][2];
        int pm0 = 0;
        uint64_t pds = 0;
        // Row offset of the previous step's tile (prow) and of this step's (row_cur), walked by
        // one row width per tile and reset to the band's first tile at each head.
        int64_t prow = 0, row_cur = 0, row0 = 0;
        if constexpr (DS) row_cur = row0 = ds_row_off(ds_bd, ur.lo >> 5);
        auto read_p = [&](int slot, f32x4* x) {
            const float* xp = &xbuf[slot][pair][0];
#pragma unroll
            for (int c = 0; c < 4; ++c) x[c] = *reinterpret_cast<const f32x4*>(xp + c * 256 + lane * 4);
        };
        auto finish = [&](const f32x4* px) {
            float pv[16];
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int e = 0; e < 4; ++e) pv[4 * c + e] = px[c][e];
            s16x8 dsb[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                float dsv[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) dsv[i] = pv[8 * kb + i] * dpm[8 * kb + i];
                u32x4 dw = {T::pack2(dsv[0], dsv[1]), T::pack2(dsv[2], dsv[3]), T::pack2(dsv[4], dsv[5]),
                            T::pack2(dsv[6], dsv[7])};
                dsb[kb] = __builtin_bit_cast(s16x8, dw);
            }
            if constexpr (DS) {
                // Block (tile pm0 / 32, key block nw0 / 32), stored only for tiles of this
                // pair's own band: the set the dS-driven dQ pass reads. Lane (key l32, g)
                // holds queries 16 kb + 8 g + 0..7 of its key (chunk ds_chunk(kb, g, l32));
                // keys past the sequence as 0.
                const int ti = pm0 >> 5;
                const int slot = ds_jblk - max(ti + ds_lob, 0);  // ds_first_block(ti, lo_f)
                const int64_t bi = prow + slot;
                if (pm0 >= wr.lo && pm0 < wr.hi && slot >= 0 && bi < ds_room) {
                    const uint64_t blk = pds + (uint64_t)bi * 2048;
                    const s16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
                    // Non-temporal: the dQ pass reads them long after; kept out of the way
                    // of the Q / dO tiles other workgroups reuse through L2 (445 -> 434 us).
                    // Keys past the sequence exist only in a sequence's last key block.
                    s16x8 d0 = dsb[0], d1 = dsb[1];
                    if (bs < 32) {
                        d0 = zero_keys ? z : d0;
                        d1 = zero_keys ? z : d1;
                    }
                    __builtin_nontemporal_store(d0, reinterpret_cast<gs16x8*>(blk + ds_lane0));
                    __builtin_nontemporal_store(d1, reinterpret_cast<gs16x8*>(blk + ds_lane1));
                }
            }
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) acc[db] = T::mfma32(qt[db][kb], dsb[kb], acc[db]);
        };
        int cur_tile = 0;
        // Unrolled by ring stage like wave A's loop; P of step it sits in xbuf[it % STAGES].
        auto b_step = [&](auto SC, int it) {
            constexpr int stage = decltype(SC)::value;
            const int m0 = ur.lo + cur_tile * BMQ;
            const uint16_t* Qs = ring + stage * STAGE;
            const uint16_t* DOs = Qs + TILE;
            const float* fl = reinterpret_cast<const float*>(Qs + 2 * TILE);
            // Operand reads first (see wave A): P of the previous tile, this tile's dO rows
            // and delta row.
            f32x4 px[4];
            if (it > 0) read_p((stage + STAGES - 1) % STAGES, px);
            s16x8 oa[KD];
#pragma unroll
            for (int kk = 0; kk < KD; ++kk) oa[kk] = lds_row_op<D>(DOs, 0, l32, g, kk);
            f32x4 dl[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) dl[c] = *reinterpret_cast<const f32x4*>(fl + 32 + 16 * (c >> 1) + 8 * g + 4 * (c & 1));
            __builtin_amdgcn_sched_barrier(0);
            if (it > 0) finish(px);
            __builtin_amdgcn_sched_barrier(0);
            pm0 = m0;
            pds = ds_ptr;
            if constexpr (DS) {
                prow = row_cur;
                row_cur = cur_tile + 1 == ntiles ? row0 : row_cur + ds_row_w(ds_bd, m0 >> 5);
            }
            if (cur_tile + 1 == ntiles) ds_ptr += ds_hstep;
            cur_tile = cur_tile + 1 == ntiles ? 0 : cur_tile + 1;
            // Q^T operands of this tile's dK product (kept for the next step), issued after the
            // previous tile's dK products have taken theirs.
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) qt[db][kb] = lds_tr_op<D>(Qs, db, kb, lane);
            // dP = dO V^T, then dP - delta in place.
            f32x16 dp;
#pragma unroll
            for (int r = 0; r < 16; ++r) dp[r] = 0.f;
#pragma unroll
            for (int kk = 0; kk < KD; ++kk) dp = T::mfma32(oa[kk], kv[kk], dp);
#pragma unroll
            for (int r = 0; r < 16; ++r) dpm[r] = dp[r] - dl[r >> 2][r & 3];
            barrier_lds();
        };
        for (int it = 0; it < iters; it += STAGES) stage_steps<0, STAGES>(b_step, it, iters);
        if (iters > 0) {
            f32x4 px[4];
            read_p((iters - 1) % STAGES, px);
            finish(px);
        }
    }

    // Sum the two head slots' partials of each key block in a fixed order (slot 1 into 0).
    if constexpr (HPW == 2) {
        float* red = reinterpret_cast<float*>(&ring_mem[0][0][0]);
        constexpr int PART = DB * 16 * 64;
        float* part_buf = red + ((role_b ? 2 : 0) + kbi) * PART;
        __syncthreads();
        if (hs == 1) {
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) part_buf[(db * 16 + r) * 64 + lane] = acc[db][r];
        }
        __syncthreads();
        if (hs == 0) {
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[db][r] += part_buf[(db * 16 + r) * 64 + lane];
        }
    }

    // Store dK * sm_scale (wave B) or dV (wave A) (flash_attn.py:312-314); lane column = key,
    // registers = d.
    if (hs == 0 && bs > 0 && key < k_len) {
        const float sc = role_b ? a.sm_scale : 1.0f;
        uint16_t* const outp = role_b ? a.dk + (int64_t)b * a.dkbs + (ks.tok0 + key) * a.dkts + (int64_t)kvh * a.dkhs
                                      : a.dv + (int64_t)b * a.dvbs + (ks.tok0 + key) * a.dvts + (int64_t)kvh * a.dvhs;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int rq = 0; rq < 4; ++rq) {
                const int d0 = 32 * db + 8 * rq + 4 * g;
                u32x2 w = {T::pack2(acc[db][4 * rq] * sc, acc[db][4 * rq + 1] * sc),
                           T::pack2(acc[db][4 * rq + 2] * sc, acc[db][4 * rq + 3] * sc)};
                *reinterpret_cast<u32x2*>(outp + d0) = w;
            }
    }
}

template <int D, int HPW, int STAGES, typename T, bool DS>
__global__ __launch_bounds__(512) void bwd_dkdv_pair_kernel(BwdArgs a) {
    dkdv_pair_block<D, HPW, STAGES, T, DS>(a, xcd_logical(blockIdx.x));
}

// The same blocks from the queues a.sched[0 .. kXcds), one persistent workgroup per CU. A
// chunk holds work iff its last rank reaches its sequence's first key block (ranks below
// gx - key blocks of the sequence hold none).
template <int D, int HPW, int STAGES, typename T>
__global__ __launch_bounds__(512) void bwd_dkdv_pair_queued_kernel(BwdArgs a) {
    constexpr int KPW = 4 / HPW;
    __shared__ Queues qs;
    const bool varlen = a.cu_k != nullptr;
    const int P = coord_pairs(a.gz, a.gy, varlen);
    const int pairs = a.gz * a.gy;
    build_queues<512>(
        qs, (a.gx + kXcdChunk - 1) / kXcdChunk * P, [&](int c) { return min(c % P / a.gz, a.gy - 1); },
        varlen ? a.cu_k : nullptr, a.seqlen_k,
        [&](int c, int k_len) { return rank_span(c / P * kXcdChunk, a.gx - (k_len + 32 * KPW - 1) / (32 * KPW), a.gx, c % P < pairs); });
    const int xcd = (int)(__smid() >> 6) & (kXcds - 1);
    int q = 0;
    for (int blk = next_block(qs, a.sched, xcd, q); blk >= 0; blk = next_block(qs, a.sched, xcd, q))
        dkdv_pair_block<D, HPW, STAGES, T, true>(fresh_args(), blk);
}

// ---- 3. dQ ------------------------------------------------------------------------------

template <int D, int BN, int NW, int STAGES, typename T>
__global__ __launch_bounds__(NW * 64) void bwd_dq_kernel(BwdArgs a) {
    constexpr int KD = D / 16;
    constexpr int DB = (D + 31) / 32;
    constexpr int NB = BN / 32;
    constexpr int KB = BN / 16;
    using Ring = TileRing<D, BN, 2, NW>;
    __shared__ __attribute__((aligned(16))) uint16_t smem[STAGES][2][BN * D];

    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int l32 = lane & 31, g = lane >> 5;
    const int tpw = NW / a.hpw;
    // Longest causal rows first across all heads and sequences, XCD-grouped.
    const BlockCoord bc = block_coord(xcd_logical(blockIdx.x), a.gz, a.gy, a.cu_q != nullptr);
    if (bc.rank >= a.gx) return;
    const int mblk = a.gx - 1 - bc.rank;
    const int h_first = bc.group * a.hpw;
    const int b = bc.seq;
    SeqInfo qs = seq_info(b, a.cu_q, nullptr, a.seqlen_q, false);
    const int tok_base = mblk * tpw * 32;
    if (tok_base >= qs.len) return;
    SeqInfo ks = seq_info(b, a.cu_k, nullptr, a.seqlen_k, false);
    const int q_len = qs.len, k_len = ks.len;
    const int kvh = h_first / a.group;
    const int lo_off = band_lo(k_len, q_len, a.wl), hi_off = band_hi(k_len, q_len, a.wr);

    int wg_lo = 1 << 30, wg_hi = 0;
    for (int tb = 0; tb < tpw; ++tb) {
        const int s0 = tok_base + tb * 32;
        const int bs = q_len - s0 < 32 ? q_len - s0 : 32;
        if (bs <= 0) continue;
        Ranges r = block_ranges(s0, bs, lo_off, hi_off, k_len, BN);
        if (r.hi > r.lo) {
            wg_lo = r.lo < wg_lo ? r.lo : wg_lo;
            wg_hi = r.hi > wg_hi ? r.hi : wg_hi;
        }
    }
    const int h = h_first + (wave % a.hpw);
    const int s0 = tok_base + (wave / a.hpw) * 32;
    const int bs = q_len - s0 < 32 ? q_len - s0 : 32;
    Ranges wr = {0, 0, 0, 0};
    if (bs > 0) wr = block_ranges(s0, bs, lo_off, hi_off, k_len, BN);

    const uint16_t* kbase = a.k + (int64_t)b * a.kbs + ks.tok0 * a.kts + (int64_t)kvh * a.khs;
    const uint16_t* vbase = a.v + (int64_t)b * a.vbs + ks.tok0 * a.vts + (int64_t)kvh * a.vhs;
    const i32x4 rsrc[2] = {rows_rsrc(kbase, k_len, a.kts, D), rows_rsrc(vbase, k_len, a.vts, D)};
    const int tstride[2] = {(int)(a.kts * 2), (int)(a.vts * 2)};

    const int qi = s0 + l32;
    const bool q_ok = bs > 0 && qi < q_len;
    s16x8 qop[KD], doop[KD];
    {
        const int64_t tokoff = qs.tok0 + qi;
        const uint16_t* qp = a.q + (int64_t)b * a.qbs + tokoff * a.qts + (int64_t)h * a.qhs;
        const uint16_t* dop = a.dout + (int64_t)b * a.dobs + tokoff * a.dots + (int64_t)h * a.dohs;
#pragma unroll
        for (int kk = 0; kk < KD; ++kk) {
            s16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
            qop[kk] = q_ok ? ld16(qp + 16 * kk + 8 * g) : z;
            doop[kk] = q_ok ? ld16(dop + 16 * kk + 8 * g) : z;
        }
    }
    // delta = rowsum(dO * O) of this wave's rows (flash_attn.py:215-216), from the dO operand
    // already in registers and the matching O chunks: lanes l32 and l32 + 32 hold the two halves
    // of a row. Written out for the dK/dV pass, which runs after this one.
    float lse_q = INFINITY, del_q = 0.f;
    {
        const uint16_t* op = a.o + (int64_t)b * a.obs + (qs.tok0 + qi) * a.ots + (int64_t)h * a.ohs;
        float part = 0.f;
#pragma unroll
        for (int kk = 0; kk < KD; ++kk) {
            s16x8 ov = {0, 0, 0, 0, 0, 0, 0, 0};
            if (q_ok) ov = ld16(op + 16 * kk + 8 * g);
#pragma unroll
            for (int i = 0; i < 8; ++i) part += T::to_float((uint16_t)ov[i]) * T::to_float((uint16_t)doop[kk][i]);
        }
        del_q = sum_halves(part);
    }
    if (q_ok) {
        const int64_t off = (int64_t)h * a.lse_hs + qs.row0 + qi;
        lse_q = a.lse[off];
        if (g == 0) a.delta[off] = del_q;
    }
    wait_vmcnt<0>();  // Q, dO, lse, delta landed before the ring's loads share the counter

    f32x16 acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;

    const int ntiles = wg_hi > wg_lo ? (wg_hi - wg_lo + BN - 1) / BN : 0;
    auto issue = [&](int t) {
        uint16_t* tiles[2] = {smem[t % STAGES][0], smem[t % STAGES][1]};
        Ring::issue(rsrc, tstride, tiles, wg_lo + t * BN, wave, lane);
    };
#pragma unroll
    for (int t = 0; t < STAGES - 1; ++t)
        if (t < ntiles) issue(t);

    for (int t = 0; t < ntiles; ++t) {
        const int n0 = wg_lo + t * BN;
        const int after = ntiles - 1 - t < STAGES - 2 ? ntiles - 1 - t : STAGES - 2;
        ring_wait<Ring::LOADS, STAGES>(after);
        barrier_lds();
        if (t + STAGES - 1 < ntiles) issue(t + STAGES - 1);
        const bool active = bs > 0 && n0 < wr.hi && n0 + BN > wr.lo;
        if (!active) continue;
        const bool masked = !(n0 >= wr.mid_lo && n0 + BN <= wr.mid_hi);
        const uint16_t* Ks = smem[t % STAGES][0];
        const uint16_t* Vs = smem[t % STAGES][1];
        // K^T operands of dQ, read first so their latency hides under the softmax work
        // (D <= 64; above, the registers are not there).
        constexpr bool PF = D <= 64;
        s16x8 kt_op[PF ? DB : 1][KB];
        if constexpr (PF) {
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int kb = 0; kb < KB; ++kb) kt_op[db][kb] = lds_tr_op<D>(Ks, db, kb, lane);
        }
        s16x8 dsb[KB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            f32x16 st, dpt;
#pragma unroll
            for (int r = 0; r < 16; ++r) st[r] = dpt[r] = 0.f;
#pragma unroll
            for (int kk = 0; kk < KD; ++kk) {
                st = T::mfma32(lds_row_op<D>(Ks, nb * 32, l32, g, kk), qop[kk], st);
                dpt = T::mfma32(lds_row_op<D>(Vs, nb * 32, l32, g, kk), doop[kk], dpt);
            }
            float dsv[16];
            if constexpr (D <= 64) {
                // P for every score first, then the band mask as one block on edge tiles only:
                // a mask test per score splits the exponentials into separately branched
                // blocks (measured 4% slower). Above D = 64 the extra live values cost a wave
                // per SIMD, so the test stays per score there.
                float pv[16];
#pragma unroll
                for (int r = 0; r < 16; ++r) pv[r] = fast_exp2(fmaf(st[r], a.qk_scale, -lse_q));
                // Key j is visible from this lane's query iff lo_off <= j - qi <= hi_off and
                // j < k_len: one range (register r holds key n0 + 32 nb + out_row32(r, g)).
                if (masked) mask_runs16(pv, n0 + nb * 32 + 8 * g, qi + lo_off, min(qi + hi_off, k_len - 1));
#pragma unroll
                for (int r = 0; r < 16; ++r) dsv[r] = pv[r] * (dpt[r] - del_q);
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float p = fast_exp2(fmaf(st[r], a.qk_scale, -lse_q));
                    if (masked) {
                        const int key = n0 + nb * 32 + out_row32(r, g);
                        const int rel = key - qi;
                        p = (rel >= lo_off && rel <= hi_off && key < k_len) ? p : 0.f;
                    }
                    dsv[r] = p * (dpt[r] - del_q);
                }
            }
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                u32x4 w = {T::pack2(dsv[8 * half], dsv[8 * half + 1]), T::pack2(dsv[8 * half + 2], dsv[8 * half + 3]),
                           T::pack2(dsv[8 * half + 4], dsv[8 * half + 5]),
                           T::pack2(dsv[8 * half + 6], dsv[8 * half + 7])};
                dsb[nb * 2 + half] = __builtin_bit_cast(s16x8, w);
            }
        }
        // dQ^T += K^T dS^T: A operand K[16 kb + 8 g + i][32 db + l32] by transpose read.
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                if constexpr (PF) acc[db] = T::mfma32(kt_op[db][kb], dsb[kb], acc[db]);
                else acc[db] = T::mfma32(lds_tr_op<D>(Ks, db, kb, lane), dsb[kb], acc[db]);
            }
    }

    if (q_ok) {
        uint16_t* dqp = a.dq + (int64_t)b * a.dqbs + (qs.tok0 + qi) * a.dqts + (int64_t)h * a.dqhs;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int rq = 0; rq < 4; ++rq) {
                const int d0 = 32 * db + 8 * rq + 4 * g;
                if (d0 < D) {
                    u32x2 w = {T::pack2(acc[db][4 * rq] * a.sm_scale, acc[db][4 * rq + 1] * a.sm_scale),
                               T::pack2(acc[db][4 * rq + 2] * a.sm_scale, acc[db][4 * rq + 3] * a.sm_scale)};
                    *reinterpret_cast<u32x2*>(dqp + d0) = w;
                }
            }
    }
}

// ---- 4. dQ from the stored dS ------------------------------------------------------------

// B operand (16 keys x 32 queries) of a 32 x 32 dS block in the ds_chunk layout in LDS: lane
// holds blk[key 16 kb + 8 g + i][query l32], i = 0..7, by two transpose reads (each 16-lane
// group: 4 keys x 16 queries, 4 consecutive queries of one key per lane).
__device__ inline s16x8 lds_tr_block32(const uint16_t* blk, int kb, int lane) {
    const int G = lane >> 4, jj = lane & 15;
    const int key = 16 * kb + 8 * (G >> 1) + (jj >> 2);
    const int qk = G & 1, qg = (jj >> 1) & 1, half = 4 * (jj & 1);
    return cat4(ds_read_tr(blk + ds_chunk(qk, qg, key) * 8 + half), ds_read_tr(blk + ds_chunk(qk, qg, key + 4) * 8 + half));
}

// dQ = sm_scale * dS K over the band from the dS blocks the dK/dV pass stored: one product per
// (query tile, key block) pair where the recomputing kernel above takes three (S and dP
// again). Workgroup = NW waves: hpw query heads of one GQA group x NW / hpw blocks of 64 query
// rows (two 32-row tiles per wave). Per step of NBK 32-key blocks a STAGES-deep direct-to-LDS
// ring brings the K rows (shared by the workgroup's heads) and each wave's 2 x NBK dS blocks
// (a block outside its tile's band is fetched through an empty buffer range, i.e. as zeros,
// so every wave issues the same loads per step). dQ^T += K^T dS^T with both operands read
// transposed. The pass streams each stored byte once: HBM-bound, except along the longest
// causal rows, whose chain of steps is covered by the ring's depth.
template <int D, int NW, int NBK, int STAGES, typename T>
__device__ __forceinline__ void dq_ds_block(const BwdArgs& a, int logical) {
    constexpr int DB = D / 32;
    constexpr int RQ = 64;
    constexpr int BN = 32 * NBK;
    using KRing = TileRing<D, BN, 1, NW>;
    constexpr int LOADS = KRing::LOADS + 4 * NBK;  // K share + 2 x NBK dS blocks of 2 KB
    constexpr int KT = BN * D;
    constexpr int DSW = 2 * NBK * 1024;            // one wave's dS blocks per stage
    constexpr int STAGE = KT + NW * DSW;
    static_assert(D % 32 == 0, "whole 32-column blocks");
    __shared__ __attribute__((aligned(16))) uint16_t smem[STAGES][STAGE];

    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int l32 = lane & 31, g = lane >> 5;
    const int hpw = a.hpw, kpw = NW / hpw;
    // Longest causal rows first across all heads and sequences, XCD-grouped.
    const BlockCoord bc = block_coord(logical, a.gz, a.gy, a.cu_q != nullptr);
    if (bc.rank >= a.gx) return;
    const int b = bc.seq;
    SeqInfo qs = seq_info(b, a.cu_q, nullptr, a.seqlen_q, false);
    const int tok_base = (a.gx - 1 - bc.rank) * kpw * RQ;
    if (tok_base >= qs.len) return;
    SeqInfo ks = seq_info(b, a.cu_k, nullptr, a.seqlen_k, false);
    const int q_len = qs.len, k_len = ks.len;
    const int hrel = bc.group * hpw + wave % hpw;  // query head within the pass
    const int h = a.kv0 * a.group + hrel;
    const int kvh = a.kv0 + bc.group * hpw / a.group;
    const int lo_f = band_lo(k_len, q_len, a.wl), hi_f = band_hi(k_len, q_len, a.wr);

    // Key range of the workgroup (union of its tiles' ranges) and this wave's two tiles.
    int wg_lo = 1 << 30, wg_hi = 0;
    for (int tt = 0; tt < 2 * kpw; ++tt) {
        const int s0 = tok_base + 32 * tt;
        const int bs = q_len - s0 < 32 ? q_len - s0 : 32;
        if (bs <= 0) break;
        const Ranges r = block_ranges(s0, bs, lo_f, hi_f, k_len, 32);
        if (r.hi > r.lo) {
            wg_lo = r.lo < wg_lo ? r.lo : wg_lo;
            wg_hi = r.hi > wg_hi ? r.hi : wg_hi;
        }
    }
    const int nsteps = wg_hi > wg_lo ? (wg_hi - wg_lo + BN - 1) / BN : 0;
    const int s_w = tok_base + (wave / hpw) * RQ;
    const int64_t ds_base = ds_seq_base(a, b);
    const DsBand ds_bd = ds_band(q_len, k_len, a.wl, a.wr);
    int blo[2], bhi[2];
    uint64_t ds_row[2];  // byte address of each tile's slot 0 minus its first block
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int s0 = s_w + 32 * tt;
        const int bs = q_len - s0 < 32 ? q_len - s0 : 32;
        blo[tt] = bhi[tt] = 0;
        const int i = s0 >> 5;
        const int64_t row = ds_base + ds_row_off(ds_bd, i);
        if (bs > 0) {
            const Ranges r = block_ranges(s0, bs, lo_f, hi_f, k_len, 32);
            const int64_t w = ds_row_w(ds_bd, i);  // the row's slots
            if (r.hi > r.lo && row + w <= a.ds_blocks) {
                blo[tt] = ds_first_block(i, lo_f);  // = r.lo / 32
                bhi[tt] = (r.hi + 31) >> 5;
                bhi[tt] = bhi[tt] - blo[tt] > w ? blo[tt] + (int)w : bhi[tt];
            }
        }
        ds_row[tt] = reinterpret_cast<uint64_t>(a.ds) +
                     (uint64_t)(((int64_t)hrel * a.ds_hs + (row - blo[tt]) * 1024) * 2);
    }

    const uint16_t* kbase = a.k + (int64_t)b * a.kbs + ks.tok0 * a.kts + (int64_t)kvh * a.khs;
    const i32x4 rsrc[1] = {rows_rsrc(kbase, k_len, a.kts, D)};
    const int tstride[1] = {(int)(a.kts * 2)};
    const int j0 = wg_lo >> 5;
    auto issue = [&](int t) {
        uint16_t* st = smem[t % STAGES];
        uint16_t* tiles[1] = {st};
        KRing::issue(rsrc, tstride, tiles, wg_lo + BN * t, wave, lane);
#pragma unroll
        for (int kb = 0; kb < NBK; ++kb) {
            const int j = j0 + NBK * t + kb;
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const bool vis = j >= blo[tt] && j < bhi[tt];
                const i32x4 r = buffer_rsrc32(ds_row[tt] + (uint64_t)j * 2048, vis ? 2048 : 0);
                const uint32_t dst = lds_addr(st + KT + wave * DSW + (kb * 2 + tt) * 1024);
                dma16_nt(r, dst, lane * 16);
                dma16_nt(r, dst + 1024, 1024 + lane * 16);
            }
        }
    };

    f32x16 acc[2][DB];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[tt][db][r] = 0.f;

#pragma unroll
    for (int t = 0; t < STAGES - 1; ++t)
        if (t < nsteps) issue(t);
    for (int t = 0; t < nsteps; ++t) {
        const int after = nsteps - 1 - t < STAGES - 2 ? nsteps - 1 - t : STAGES - 2;
        ring_wait<LOADS, STAGES>(after);
        barrier_lds();
        if (t + STAGES - 1 < nsteps) issue(t + STAGES - 1);
        const uint16_t* Ks = smem[t % STAGES];
        const uint16_t* Ds = Ks + KT + wave * DSW;
#pragma unroll
        for (int kb = 0; kb < NBK; ++kb) {
            const int j = j0 + NBK * t + kb;
            const bool v0 = j >= blo[0] && j < bhi[0], v1 = j >= blo[1] && j < bhi[1];
            if (!(v0 || v1)) continue;
            s16x8 kt[DB][2];
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) kt[db][kk] = lds_tr_op<D>(Ks, db, 2 * kb + kk, lane);
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                if (!(tt == 0 ? v0 : v1)) continue;
                const uint16_t* blk = Ds + (kb * 2 + tt) * 1024;
                const s16x8 d0 = lds_tr_block32(blk, 0, lane);
                const s16x8 d1 = lds_tr_block32(blk, 1, lane);
#pragma unroll
                for (int db = 0; db < DB; ++db) {
                    acc[tt][db] = T::mfma32(kt[db][0], d0, acc[tt][db]);
                    acc[tt][db] = T::mfma32(kt[db][1], d1, acc[tt][db]);
                }
            }
        }
    }

    // dQ^T rows = d (registers), columns = queries (lanes): 8-byte stores of 4 consecutive d.
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int qi = s_w + 32 * tt + l32;
        if (qi >= q_len) continue;
        uint16_t* dqp = a.dq + (int64_t)b * a.dqbs + (qs.tok0 + qi) * a.dqts + (int64_t)h * a.dqhs;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int rq = 0; rq < 4; ++rq) {
                const int d0 = 32 * db + 8 * rq + 4 * g;
                const f32x16& c = acc[tt][db];
                u32x2 w = {T::pack2(c[4 * rq] * a.sm_scale, c[4 * rq + 1] * a.sm_scale),
                           T::pack2(c[4 * rq + 2] * a.sm_scale, c[4 * rq + 3] * a.sm_scale)};
                *reinterpret_cast<u32x2*>(dqp + d0) = w;
            }
    }
}

template <int D, int NW, int NBK, int STAGES, typename T>
__global__ __launch_bounds__(NW * 64) void bwd_dq_ds_kernel(BwdArgs a) {
    dq_ds_block<D, NW, NBK, STAGES, T>(a, xcd_logical(blockIdx.x));
}

int gcd_int(int x, int y) {
    while (y) {
        int t = x % y;
        x = y;
        y = t;
    }
    return x;
}

// Workgroups of a queued launch: per_cu per CU of the current device (a count read once per
// device). More than can be resident is harmless: every workgroup drains the queues.
int queued_grid(int per_cu) {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256 * per_cu;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev] * per_cu;
}

BwdArgs make_args(const mykfa_bwd_params& p) {
    const mykfa_fwd_params& f = p.fwd;
    BwdArgs a;
    a.q = static_cast<const uint16_t*>(f.q);
    a.k = static_cast<const uint16_t*>(f.k);
    a.v = static_cast<const uint16_t*>(f.v);
    a.o = static_cast<const uint16_t*>(f.o);
    a.dout = static_cast<const uint16_t*>(p.dout);
    a.dq = static_cast<uint16_t*>(p.dq);
    a.dk = static_cast<uint16_t*>(p.dk);
    a.dv = static_cast<uint16_t*>(p.dv);
    a.lse = f.lse;
    a.delta = p.delta;
    a.qbs = f.q_batch_stride; a.qts = f.q_token_stride; a.qhs = f.q_head_stride;
    a.kbs = f.k_batch_stride; a.kts = f.k_token_stride; a.khs = f.k_head_stride;
    a.vbs = f.v_batch_stride; a.vts = f.v_token_stride; a.vhs = f.v_head_stride;
    a.obs = f.o_batch_stride; a.ots = f.o_token_stride; a.ohs = f.o_head_stride;
    a.dobs = p.do_batch_stride; a.dots = p.do_token_stride; a.dohs = p.do_head_stride;
    a.dqbs = p.dq_batch_stride; a.dqts = p.dq_token_stride; a.dqhs = p.dq_head_stride;
    a.dkbs = p.dk_batch_stride; a.dkts = p.dk_token_stride; a.dkhs = p.dk_head_stride;
    a.dvbs = p.dv_batch_stride; a.dvts = p.dv_token_stride; a.dvhs = p.dv_head_stride;
    a.lse_hs = f.lse_head_stride;
    a.cu_q = f.cu_seqlens_q;
    a.cu_k = f.cu_seqlens_k;
    a.seqlen_q = f.max_seqlen_q;
    a.seqlen_k = f.max_seqlen_k;
    a.wl = f.window_left;
    a.wr = f.window_right;
    a.qk_scale = f.softmax_scale * 1.4426950408889634f;
    a.sm_scale = f.softmax_scale;
    a.group = f.num_heads / f.num_kv_heads;
    a.hpw = 1;  // set per kernel shape by its launcher
    a.num_heads = f.num_heads;
    a.batch = f.batch;
    a.ds = nullptr;
    a.ds_hs = 0;
    a.ds_blocks = 0;
    a.ds_base = nullptr;
    a.ds_seq_dense = 0;
    a.kv0 = 0;
    a.sched = nullptr;
    a.sched_zero = 0;
    return a;
}

template <typename T>
hipError_t preprocess_dtype(const BwdArgs& a, int D, hipStream_t s) {
    // Items = rows x heads over at most the rows the launch covers (the varlen row count is
    // read on the device); enough blocks for every lane to keep U items in flight once.
    const long long rows = (long long)a.batch * a.seqlen_q;
    const long long items = rows * a.num_heads;
    const long long per_block = (256 / (D / 8)) * 4;
    long long blocks = (items + per_block - 1) / per_block;
    blocks = blocks < 1 ? 1 : (blocks > 8192 ? 8192 : blocks);
    dim3 grid((unsigned)blocks);
    switch (D) {
        case 16: hipLaunchKernelGGL((bwd_delta_kernel<16, T>), grid, dim3(256), 0, s, a); break;
        case 32: hipLaunchKernelGGL((bwd_delta_kernel<32, T>), grid, dim3(256), 0, s, a); break;
        case 64: hipLaunchKernelGGL((bwd_delta_kernel<64, T>), grid, dim3(256), 0, s, a); break;
        case 128: hipLaunchKernelGGL((bwd_delta_kernel<128, T>), grid, dim3(256), 0, s, a); break;
        case 256: hipLaunchKernelGGL((bwd_delta_kernel<256, T>), grid, dim3(256), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int D, int NW, int STAGES, typename T, bool DS = false>
hipError_t dkdv_launch(BwdArgs a, int num_kv_heads, hipStream_t s) {
    a.hpw = gcd_int(a.group, NW);
    const int keys_per_wg = 32 * (NW / a.hpw);
    a.gx = (a.seqlen_k + keys_per_wg - 1) / keys_per_wg;
    a.gy = a.batch;
    a.gz = num_kv_heads;
    const long long n = block_grid_size(a.gx, a.gz, a.gy, a.cu_k != nullptr);
    if (n == 0) return hipSuccess;
    if (n > (1LL << 30)) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((bwd_dkdv_kernel<D, NW, STAGES, T, DS>), dim3(xcd_grid((int)n)), dim3(NW * 64), 0, s, a);
    return hipGetLastError();
}

// Wave-pair dK/dV: HPW = 2 query heads x 2 key blocks per workgroup when the GQA group is
// even, else 1 head x 4 key blocks.
template <int D, int HPW, int STAGES, typename T, bool DS>
hipError_t dkdv_pair_launch_hpw(BwdArgs a, int num_kv_heads, hipStream_t s) {
    a.hpw = HPW;
    const int keys_per_wg = 32 * (4 / HPW);
    a.gx = (a.seqlen_k + keys_per_wg - 1) / keys_per_wg;
    a.gy = a.batch;
    a.gz = num_kv_heads;
    const long long n = block_grid_size(a.gx, a.gz, a.gy, a.cu_k != nullptr);
    if (n == 0) return hipSuccess;
    if (n > (1LL << 30)) return hipErrorInvalidConfiguration;
    if (DS && a.sched != nullptr && n / kXcdChunk <= kQueueCap) {
        hipLaunchKernelGGL((bwd_dkdv_pair_queued_kernel<D, HPW, STAGES, T>), dim3(queued_grid(1)), dim3(512), 0, s, a);
        return hipGetLastError();
    }
    hipLaunchKernelGGL((bwd_dkdv_pair_kernel<D, HPW, STAGES, T, DS>), dim3(xcd_grid((int)n)), dim3(512), 0, s, a);
    return hipGetLastError();
}
template <int D, typename T, bool DS = false>
hipError_t dkdv_pair_launch(const BwdArgs& a, int num_kv_heads, hipStream_t s) {
    if (a.group % 2 == 0) return dkdv_pair_launch_hpw<D, 2, 3, T, DS>(a, num_kv_heads, s);
    return dkdv_pair_launch_hpw<D, 1, 4, T, DS>(a, num_kv_heads, s);
}
// MYKFA_DKDV_PAIR=0 selects the single-wave dK/dV kernel at head_dim 128 (for comparisons; at
// head_dim 64 the single-wave kernel is the faster one: cfg2 dK/dV 63.9 us against 83.5 us for
// the pair kernel, whose per-step exchange and barrier do not shrink with D).
bool dkdv_pair_enabled() {
    static const bool on = [] {
        const char* e = getenv("MYKFA_DKDV_PAIR");
        return e == nullptr || e[0] != '0';
    }();
    return on;
}
template <typename T>
hipError_t dkdv_dtype(const BwdArgs& a, int D, int num_kv_heads, hipStream_t s) {
    switch (D) {
        case 16: return dkdv_launch<16, 4, 3, T>(a, num_kv_heads, s);
        case 32: return dkdv_launch<32, 4, 3, T>(a, num_kv_heads, s);
        case 64: return dkdv_launch<64, 4, 2, T>(a, num_kv_heads, s);
        case 128:
            if (dkdv_pair_enabled()) return dkdv_pair_launch<128, T>(a, num_kv_heads, s);
            return dkdv_launch<128, 4, 2, T>(a, num_kv_heads, s);
        case 256: return dkdv_launch<256, 2, 2, T>(a, num_kv_heads, s);
        default: return hipErrorInvalidValue;
    }
}

template <int D, int BN, int NW, int STAGES, typename T>
hipError_t dq_launch(BwdArgs a, hipStream_t s) {
    a.hpw = gcd_int(a.group, NW);
    const int tpw = NW / a.hpw;
    a.gx = (a.seqlen_q + tpw * 32 - 1) / (tpw * 32);
    a.gy = a.batch;
    a.gz = a.num_heads / a.hpw;
    const long long n = block_grid_size(a.gx, a.gz, a.gy, a.cu_q != nullptr);
    if (n == 0) return hipSuccess;
    if (n > (1LL << 30)) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((bwd_dq_kernel<D, BN, NW, STAGES, T>), dim3(xcd_grid((int)n)), dim3(NW * 64), 0, s, a);
    return hipGetLastError();
}

template <typename T>
hipError_t dq_dtype(const BwdArgs& a, int D, hipStream_t s) {
    switch (D) {
        case 16: return dq_launch<16, 64, 4, 4, T>(a, s);
        case 32: return dq_launch<32, 64, 4, 4, T>(a, s);
        // 64-key steps in 2 stages: half the steps (barriers, ring waits) of 32-key steps on the
        // longest causal rows; cfg2 dQ 51.9 -> 49.9 us (32 keys in 3, 4 or 6 stages and 64
        // keys in 3 stages measured slower).
        case 64: return dq_launch<64, 64, 4, 2, T>(a, s);
        case 128: return dq_launch<128, 64, 4, 2, T>(a, s);
        case 256: return dq_launch<256, 32, 4, 3, T>(a, s);
        default: return hipErrorInvalidValue;
    }
}

// dS-driven dQ over the pass's num_kv_heads KV heads (a.kv0 on).
template <int D, int NW, int NBK, int STAGES, typename T>
hipError_t dq_ds_launch(BwdArgs a, int num_kv_heads, hipStream_t s) {
    a.hpw = gcd_int(a.group, NW);
    const int rows_per_wg = 64 * (NW / a.hpw);
    a.gx = (a.seqlen_q + rows_per_wg - 1) / rows_per_wg;
    a.gy = a.batch;
    a.gz = num_kv_heads * a.group / a.hpw;
    const long long n = block_grid_size(a.gx, a.gz, a.gy, a.cu_q != nullptr);
    if (n == 0) return hipSuccess;
    if (n > (1LL << 30)) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((bwd_dq_ds_kernel<D, NW, NBK, STAGES, T>), dim3(xcd_grid((int)n)), dim3(NW * 64), 0, s, a);
    return hipGetLastError();
}

// Delta, then per pass of kv_per_pass KV heads: dK/dV storing dS, and dQ from dS.
template <typename T>
hipError_t ds_passes(BwdArgs a, const mykfa_bwd_params& p, int kv_per_pass, hipStream_t s) {
    // Queue counters after the pass's dS (kSchedBytes per KV head of the pass), a set per
    // pass, zeroed by the delta kernel.
    const int passes = (p.fwd.num_kv_heads + kv_per_pass - 1) / kv_per_pass;
    int* const sched = reinterpret_cast<int*>(a.ds + (int64_t)kv_per_pass * a.group * a.ds_hs);
    const bool queued = (size_t)passes * kQueueSet * sizeof(int) <= (size_t)kv_per_pass * kSchedBytes;
    a.sched = queued ? sched : nullptr;
    a.sched_zero = queued ? passes * kQueueSet : 0;
    hipError_t e = preprocess_dtype<T>(a, p.fwd.head_dim, s);
    for (int kv0 = 0; e == hipSuccess && kv0 < p.fwd.num_kv_heads; kv0 += kv_per_pass) {
        const int n = p.fwd.num_kv_heads - kv0 < kv_per_pass ? p.fwd.num_kv_heads - kv0 : kv_per_pass;
        a.kv0 = kv0;
        a.sched = queued ? sched + (kv0 / kv_per_pass) * kQueueSet : nullptr;
        // dQ: 64 keys per step, 3 stages (144 KB of LDS: one workgroup per CU) measured best
        // among 32 / 64 keys per step and 2-6 stages (the single-workgroup ring holds the most
        // bytes in flight).
        e = dkdv_pair_enabled() ? dkdv_pair_launch<128, T, true>(a, n, s) : dkdv_launch<128, 4, 2, T, true>(a, n, s);
        if (e == hipSuccess) e = dq_ds_launch<128, 4, 2, 3, T>(a, n, s);
    }
    return e;
}

// Blocks per query head of the compact dS layout. Dense batches: exact. Packed batches: the
// host knows only the packed row count T (lse_head_stride), the batch B and max_seqlen, so the
// size is an upper bound over all length distributions: at most (T + 31 B) / 32 query tiles,
// each with at most the widest band's slots; and for causal self-attention (cu_seqlens_q ==
// cu_seqlens_k, right window 0) a tile's row widths grow along its sequence (1, 2, ... up to
// the window), so a sequence's mean row width grows with its length and no batch exceeds the
// tiles times the mean width of a max_seqlen sequence (cfg3: 337 MB per KV head where rows of
// the longest sequence's width took 673 MB; 164 MB are written).
int64_t ds_head_blocks(const mykfa_fwd_params& f) {
    const int wl = f.window_left, wr = f.window_right;
    if (f.cu_seqlens_q == nullptr) return (int64_t)f.batch * ds_seq_blocks(f.max_seqlen_q, f.max_seqlen_k, wl, wr);
    const int64_t tiles = (f.lse_head_stride + 31LL * f.batch) / 32;
    const int64_t all = (f.max_seqlen_k + 31) / 32;
    const int64_t band = (32 + (int64_t)wl + wr + 31) / 32 + 1;
    const int64_t rect = tiles * (all < band ? all : band);
    if (f.cu_seqlens_q != f.cu_seqlens_k || wr != 0) return rect;
    const int M = f.max_seqlen_q < f.max_seqlen_k ? f.max_seqlen_q : f.max_seqlen_k;
    const int64_t ntM = (M + 31) / 32;
    if (ntM <= 0) return rect;
    const int64_t tri = (tiles * ds_seq_blocks(M, M, wl, wr) + ntM - 1) / ntM;
    return tri < rect ? tri : rect;
}
// Bytes of the packed batch's sequence-start table (batch + 1 int64), 256-byte granular.
size_t ds_table_bytes(const mykfa_fwd_params& f) {
    return f.cu_seqlens_q == nullptr ? 0 : ((size_t)(f.batch + 1) * 8 + 255) / 256 * 256;
}

}  // namespace

size_t bwd_ds_bytes_per_kv_head(const mykfa_bwd_params& p) {
    const mykfa_fwd_params& f = p.fwd;
    // Only head_dim 128: at 64 the dK/dV pass's stores and the separate delta pass cost more
    // than the recomputed S and dP they save (measured on packed and dense batches).
    if (f.head_dim != 128) return 0;
    if (f.batch <= 0 || f.max_seqlen_q <= 0 || f.max_seqlen_k <= 0) return 0;
    const int64_t group = f.num_heads / f.num_kv_heads;
    return (size_t)(group * ds_head_blocks(f)) * 2048 + kSchedBytes + ds_table_bytes(f);
}

// Workspace of kv_heads KV heads' worth: their dS, then their block-queue counters, then the
// sequence-start table.
BwdArgs ds_args(const mykfa_bwd_params& p, void* ws, int kv_heads) {
    BwdArgs a = make_args(p);
    a.ds = static_cast<uint16_t*>(ws);
    a.ds_blocks = ds_head_blocks(p.fwd);
    a.ds_hs = a.ds_blocks * 1024;
    a.ds_seq_dense = p.fwd.cu_seqlens_q == nullptr ? ds_seq_blocks(p.fwd.max_seqlen_q, p.fwd.max_seqlen_k,
                                                                   p.fwd.window_left, p.fwd.window_right)
                                                   : 0;
    char* tail = static_cast<char*>(ws) + (size_t)kv_heads * ((size_t)a.group * a.ds_hs * 2 + kSchedBytes);
    a.ds_base = p.fwd.cu_seqlens_q != nullptr ? reinterpret_cast<const int64_t*>(tail) : nullptr;
    return a;
}

hipError_t launch_bwd_ds(const mykfa_bwd_params& p, void* ws, int kv_per_pass, hipStream_t stream) {
    const BwdArgs a = ds_args(p, ws, kv_per_pass);
    if (p.fwd.dtype == MYKFA_BF16) return ds_passes<BF16>(a, p, kv_per_pass, stream);
    return ds_passes<FP16>(a, p, kv_per_pass, stream);
}

hipError_t launch_bwd_ds_half(const mykfa_bwd_params& p, void* ws, bool dq, hipStream_t stream) {
    const int n = p.fwd.num_kv_heads;
    BwdArgs a = ds_args(p, ws, n);
    // One pass over every KV head: its queue counters after the dS, zeroed here, and the
    // sequence-start table (the same in both halves).
    a.sched = reinterpret_cast<int*>(a.ds + (int64_t)n * a.group * a.ds_hs);
    a.sched_zero = kQueueSet;
    hipLaunchKernelGGL(sched_zero_kernel, dim3(1), dim3(64), 0, stream, a);
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    const bool pair = dkdv_pair_enabled();
    if (p.fwd.dtype == MYKFA_BF16) {
        if (dq) return dq_ds_launch<128, 4, 2, 3, BF16>(a, n, stream);
        return pair ? dkdv_pair_launch<128, BF16, true>(a, n, stream) : dkdv_launch<128, 4, 2, BF16, true>(a, n, stream);
    }
    if (dq) return dq_ds_launch<128, 4, 2, 3, FP16>(a, n, stream);
    return pair ? dkdv_pair_launch<128, FP16, true>(a, n, stream) : dkdv_launch<128, 4, 2, FP16, true>(a, n, stream);
}

hipError_t launch_bwd_preprocess(const mykfa_bwd_params& p, hipStream_t stream) {
    BwdArgs a = make_args(p);
    if (p.fwd.dtype == MYKFA_BF16) return preprocess_dtype<BF16>(a, p.fwd.head_dim, stream);
    return preprocess_dtype<FP16>(a, p.fwd.head_dim, stream);
}

hipError_t launch_bwd_dkdv(const mykfa_bwd_params& p, hipStream_t stream) {
    BwdArgs a = make_args(p);
    if (p.fwd.dtype == MYKFA_BF16) return dkdv_dtype<BF16>(a, p.fwd.head_dim, p.fwd.num_kv_heads, stream);
    return dkdv_dtype<FP16>(a, p.fwd.head_dim, p.fwd.num_kv_heads, stream);
}

hipError_t launch_bwd_dq(const mykfa_bwd_params& p, hipStream_t stream) {
    BwdArgs a = make_args(p);
    if (p.fwd.dtype == MYKFA_BF16) return dq_dtype<BF16>(a, p.fwd.head_dim, stream);
    return dq_dtype<FP16>(a, p.fwd.head_dim, stream);
}

}  // namespace mykfa
