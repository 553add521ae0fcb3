// KV-cache decode: split-K forward over the cache length plus an LSE merge, and the KV
// append (replaces the decode configuration of _fwd_kernel, flash_attn.py:324, :364, and
// the cache writes of flash_attn_with_kvcache, flash_attn.py:480-488).
//
// Rows. All GROUP query heads of one KV head and all seqlen_q queries are packed as the
// rows of one 16-row MFMA tile (row = head_in_group * seqlen_q + query), so each K/V byte
// is read from HBM once per GQA group, not once per query head. With GROUP = 4 and the
// 4-query MTP draft this exactly fills the tile.
//
// Split-K, balanced by length. A split-K pass takes as long as its most loaded CU: with splits
// sized from the cache capacity (the host knows no lengths) a batch of random lengths left
// half the workgroups empty and some CUs with two full splits (measured on 64 sequences of
// U[256, 16384] keys: 74-107 us for the same bytes depending only on where split boundaries
// fell). So every workgroup first reads the sequences' lengths and computes the same plan on
// the device: a chunk target T from the total visible keys such that the active workgroups fit
// one resident round, s_b = ceil(V_b / T) equal splits for sequence b, numbered sequence by
// sequence; workgroup x takes split x of that numbering (assign_split). Each covers its split's
// keys for kWaves consecutive (KV head, row tile) units, one per wave, so the waves of a
// workgroup read adjacent heads of the same cache rows (contiguous DRAM rows in the usual
// (batch, token, head, d) layout) and share nothing after the plan: no cross-wave merge.
// A wave streams its keys in 32-key tiles through a ring of NBUF register tiles filled by
// bounds-checked buffer loads (NBUF - 1 tiles in flight while one computes). Every load reads
// whole 128-byte lines (8 lanes per key row of 64 elements): a load in the MFMA operand layout
// itself would read 16 keys x 64 bytes, two requests per line, which measured 8% slower at the
// same bytes. The tile then goes through wave-private LDS: K is read back as the A operand of
// S^T = K Q^T on 16x16x32 MFMA, then the online softmax, and V is read back transposed for
// O^T += V^T P^T. A wave then
// writes either the final O/LSE (a sequence of one split) or an fp32 partial (O, lse) that the
// merge kernel combines: lse = log2(sum_s 2^lse_s), O = sum_s 2^(lse_s - lse) O_s.
#include <mutex>

#include "common.h"
#include "kernels.h"

namespace mykfa {

// Split-K workspace of the allocation-free decode entry point (mykfa_decode_noalloc): a
// file-scope device array, one copy per GPU the library runs on, held until the process ends.
// Host code never uses this name as an address (in host code it is only a stand-in for the
// device symbol): decode_scratch() resolves each device's copy once with hipGetSymbolAddress
// and every launch passes that pointer.
static __device__ __align__(256) unsigned char scratch[MYKFA_DECODE_SCRATCH_BYTES];

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
    int units;     // num_kv_heads * row_tiles (one wave each)
    int num_heads;
    int nseg;      // partial segments the workspace holds: slots per sequence * batch
    int resident;  // workgroups the chip holds at once (the balance target)
    int n_new;     // keys appended after seqused_k[b] in this step
    const uint16_t* kn;  // new keys / values to write into the caches first, or null
    const uint16_t* vn;
    int64_t knbs, knts, knhs, vnbs, vnts, vnhs;
    // Partials of segment = (first segment of the sequence) + split. A partial O is the
    // normalized output of its split, a convex combination of V rows, so it is stored in the
    // 16-bit input type (it cannot leave V's range); the lse stays fp32.
    uint16_t* ws_o;  // [nseg][num_heads][nq][D]
    float* ws_lse;   // [nseg][num_heads][nq]
    int* seg_hdr;  // [batch][2]: first segment and split count of each sequence, for the merge
    int batch;
};

// Keys of sequence b (cached plus this step's new ones), clamped to the cache capacity so
// no read leaves the cache.
__device__ inline int seq_keys(const DecodeArgs& a, int b) {
    if (!a.seqused_k) return a.cap;
    const int L = a.seqused_k[b] + a.n_new;
    return L < 0 ? 0 : (L > a.cap ? a.cap : L);
}

// Keys any row of sequence b can see, as a kTile-aligned [lo, hi) (flash_attn.py:58-68 with
// the queries as the self block).
__device__ inline Ranges decode_ranges(const DecodeArgs& a, int L) {
    const int lo_off = band_lo(L, a.nq, a.wl), hi_off = band_hi(L, a.nq, a.wr);
    return block_ranges(0, a.nq, lo_off, hi_off, L, kTile);
}

// Register ring depth (32-key tiles of K and V in flight per wave) by head_dim: one tile
// holds 2 * 32 * D bytes in 32 * D / 64 * 2 / 4 VGPRs.
template <int D>
constexpr int decode_nbuf() { return D <= 64 ? 3 : 2; }  // measured at D = 64: 3 > 4 > 6 tiles

// Visible keys of sequence b: the kTile-aligned range any of its rows can see.
__device__ inline int visible_keys(const DecodeArgs& a, int b) {
    const Ranges rg = decode_ranges(a, seq_keys(a, b));
    return rg.hi > rg.lo ? rg.hi - rg.lo : 0;
}

// Keys per split of the length-balanced split-K (a multiple of kTile) for K visible keys in
// all: the launch's active workgroups should fit one resident round of the chip (a.resident
// workgroup slots), since a split-K pass takes as long as its most loaded CU. Sequence b then
// takes s_b = max(1, ceil(V_b / T)) splits of ceil(V_b / s_b) keys; with A the target count,
// sum s_b <= K / T + batch <= A + batch <= a.nseg, so the segments always fit the workspace.
__device__ inline int balanced_chunk(const DecodeArgs& a, long long K) {
    if (a.nseg <= a.batch) return 1 << 30;  // one slot per sequence: one split each
    long long A = (long long)min(a.resident, a.nseg) - a.batch;
    if (A < 1) A = a.nseg - a.batch;
    long long T = (K + A - 1) / A;
    T = (T + kTile - 1) / kTile * kTile;
    return (int)(T < kTile ? kTile : (T > (1 << 30) ? (1 << 30) : T));
}

// Splits of a sequence with V visible keys under chunk target T.
__device__ inline int seq_splits(int V, int T) { return V > T ? (V + T - 1) / T : 1; }

// Keys the split holding a step's appended keys gives up to the other splits of its sequence.
constexpr int kOwnerShort = 384;

struct SplitOf {
    int b;      // sequence, or -1 when the workgroup holds no split
    int split;  // index of the split within the sequence
    int n;      // splits of the sequence
    int seg;    // workspace segment of split 0 (segments of a sequence are consecutive)
    int chunk;  // keys per split of the sequence (a multiple of kTile)
};

// Workgroup w's split of the length-balanced split-K: the sequences' visible key counts V_b
// are read on the device (every workgroup computes the same plan), T follows from their sum
// (balanced_chunk), and the splits are numbered sequence by sequence, so workgroup w takes the
// split whose running index is w; workgroups beyond the last split exit. The first batch
// workgroups (of z-slice 0) also record (first segment, splits) of sequence w for the merge.
// Block-uniform call: every thread of the workgroup takes part (two passes over the batch,
// NT sequences at a time, with block-wide reductions through `red`).
template <int NT>
__device__ SplitOf assign_split(const DecodeArgs& a, int w, bool write_header, int* red) {
    constexpr int NW = NT / 64;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    // Pass 1: K = sum of V_b. One register holds V_b when the batch fits one pass.
    int v_keep = 0;
    long long kpart = 0;
    for (int b0 = 0; b0 < a.batch; b0 += NT) {
        const int b = b0 + tid;
        const int v = b < a.batch ? visible_keys(a, b) : 0;
        if (b0 == 0) v_keep = v;
        kpart += v;
    }
    long long* redll = reinterpret_cast<long long*>(red);
    auto block_sum = [&](long long x) {
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
        if (lane == 0) redll[wv] = x;
        __syncthreads();
        long long t = 0;
#pragma unroll
        for (int i = 0; i < NW; ++i) t += redll[i];
        __syncthreads();
        return t;
    };
    // (Filling the slots more closely, with a smaller target that a count of the actual
    // splits allows, measured slower: 501 active workgroups took 83.2 us where 476 took 81.2.)
    const int T = balanced_chunk(a, block_sum(kpart));
    // Pass 2: exclusive scan of s_b; the thread whose sequence holds split w records it.
    SplitOf r = {-1, 0, 0, 0, 0};
    int* slot = red + 2 * NW;  // [0..4]: the found split
    if (tid == 0) slot[0] = -1;
    int run = 0;
    for (int b0 = 0; b0 < a.batch; b0 += NT) {
        const int b = b0 + tid;
        const int v = b < a.batch ? (b0 == 0 ? v_keep : visible_keys(a, b)) : 0;
        const int s = b < a.batch ? seq_splits(v, T) : 0;
        int inc = s;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int y = __shfl_up(inc, off);
            if (lane >= off) inc += y;
        }
        if (lane == 63) red[wv] = inc;
        __syncthreads();
        int before = run, tot = 0;
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            before += i < wv ? red[i] : 0;
            tot += red[i];
        }
        const int seg0 = before + inc - s;
        if (b < a.batch) {
            if (w >= seg0 && w < seg0 + s) {
                const int c = (v + s - 1) / s;
                slot[0] = b;
                slot[1] = w - seg0;
                slot[2] = s;
                slot[3] = seg0;
                int ck = c < kTile ? kTile : (c + kTile - 1) / kTile * kTile;
                // Splits start ck cache rows apart; power-of-two distances put concurrently
                // starting workgroups on the same DRAM channels (measured ~15% slower).
                if (ck > kTile && (ck & (ck - 1)) == 0) ck += kTile;
                if (a.kn != nullptr && s > 1) {
                    // The last split also stores this step's new keys and waits for those
                    // stores before its loads: it gets kOwnerShort fewer keys than the others
                    // (as long as a tile is left), so that it does not end last (64 x 16K-cache
                    // batch, one query and the 4-query draft: 1.4-2.1 us less per layer for 160 to
                    // 512 keys, 2.1 at 384).
                    const int c2 = (v + kOwnerShort + s - 1) / s;
                    int ck2 = (c2 + kTile - 1) / kTile * kTile;
                    if (ck2 > kTile && (ck2 & (ck2 - 1)) == 0) ck2 += kTile;
                    if (v - (s - 1) * ck2 >= kTile) ck = ck2;
                }
                slot[4] = ck;
            }
            if (write_header && b == w) {
                a.seg_hdr[2 * b] = seg0;
                a.seg_hdr[2 * b + 1] = s;
            }
        }
        run += tot;
        __syncthreads();
    }
    r.b = slot[0];
    if (r.b >= 0) {
        r.split = slot[1];
        r.n = slot[2];
        r.seg = slot[3];
        r.chunk = slot[4];
    }
    return r;
}

template <int D, typename T>
__global__ __launch_bounds__(kThreads) void decode_splitk_kernel(DecodeArgs a) {
    constexpr int KD = D < 32 ? 1 : D / 32;  // 32-wide d steps of S^T (D = 16 pads to 32)
    constexpr int DB = (D + 15) / 16;        // 16-row blocks of O^T
    constexpr int VPL = kTile * D / 8 / 64;  // 16-byte chunks per lane of a K or V tile
    constexpr int NBUF = decode_nbuf<D>();
    static_assert(kTile * D / 8 >= 64 && (kTile * D / 8) % 64 == 0, "K/V tile is whole 64-lane loads");
    // Staging: double-buffered up to D = 64 (16 KB per wave), single above so that two
    // workgroups still fit a CU (LDS ops of one wave execute in order, so one buffer is safe).
    constexpr int NPAR = D <= 64 ? 2 : 1;
    __shared__ __attribute__((aligned(16))) uint16_t klds[kWaves][NPAR][kTile * D];
    __shared__ __attribute__((aligned(16))) uint16_t vlds[kWaves][NPAR][kTile * D];

    const int tid = __builtin_amdgcn_workitem_id_x();
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int l16 = lane & 15, G = lane >> 4;
    // Workgroup (x, 0, z) = split x of the launch's running split index (assign_split) for
    // kWaves consecutive (KV head, row tile) units z * kWaves ..; one unit per wave: the waves of
    // a workgroup read adjacent heads of the same cache rows and share nothing after the plan.
    __shared__ int plan_red[2 * kWaves + 5];
    const SplitOf so = assign_split<kThreads>(a, blockIdx.x, blockIdx.z == 0 && a.seg_hdr != nullptr, plan_red);
    if (so.b < 0) return;
    const int split = so.split, b = so.b;
    const int unit = blockIdx.z * kWaves + wave;
    if (unit >= a.units) return;
    const int kvh = unit / a.row_tiles, rt = unit % a.row_tiles;

    const int L = seq_keys(a, b);
    const Ranges rg = decode_ranges(a, L);
    const int k0 = rg.lo + split * so.chunk;
    const int k1 = k0 + so.chunk < rg.hi ? k0 + so.chunk : rg.hi;  // k1 <= k0 only for an empty sequence
    const int lo_off = band_lo(L, a.nq, a.wl), hi_off = band_hi(L, a.nq, a.wr);

    // Q^T operand: lane holds Q[row l16][32 kk + 8 G + i]. Issued before the appended keys'
    // loads, so that their latencies overlap (the stores wait for the new keys' data).
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
    if (a.kn) {
        // This step's new keys first (flash_attn.py:480-485): the wave writes the rows of its KV
        // head that fall in its split's key range (rows before the visible range go to split 0),
        // whatever their visibility, and drops rows at or beyond the capacity. Every wave
        // reading a row wrote it itself (waves of further row tiles of a head write identical
        // copies), and the wait below orders its stores before its loads.
        const int base = a.seqused_k[b];
        constexpr int CPR = D / 8;
        for (int i = lane; i < a.n_new * CPR; i += 64) {
            const int t = i / CPR, ch = i % CPR;
            const int pos = base + t;
            const int owner = pos < rg.lo ? 0 : min((pos - rg.lo) / so.chunk, so.n - 1);
            if (pos < 0 || pos >= a.cap || owner != split) continue;
            const int64_t src_k = (int64_t)b * a.knbs + (int64_t)t * a.knts + (int64_t)kvh * a.knhs + ch * 8;
            const int64_t src_v = (int64_t)b * a.vnbs + (int64_t)t * a.vnts + (int64_t)kvh * a.vnhs + ch * 8;
            const int64_t dst_k = (int64_t)b * a.kbs + (int64_t)pos * a.kts + (int64_t)kvh * a.khs + ch * 8;
            const int64_t dst_v = (int64_t)b * a.vbs + (int64_t)pos * a.vts + (int64_t)kvh * a.vhs + ch * 8;
            st16(const_cast<uint16_t*>(a.k) + dst_k, ld16(a.kn + src_k));
            st16(const_cast<uint16_t*>(a.v) + dst_v, ld16(a.vn + src_v));
        }
    }
    // Q landed (and any appended rows stored) before the ring's loads share the in-order
    // counter; otherwise the counter analysis cannot bound the loop's pending loads and drains
    // them at the loop head.
    wait_vmcnt<0>();

    // K / V rows 0 .. L-1 of this (sequence, KV head) through bounds-checked buffer loads: keys
    // at or beyond L read 0 and a load whose offset is at or above 2^31 fetches nothing, which
    // is how tiles past the split's end are skipped without a branch.
    const uint16_t* kbase = a.k + (int64_t)b * a.kbs + (int64_t)kvh * a.khs;
    const uint16_t* vbase = a.v + (int64_t)b * a.vbs + (int64_t)kvh * a.vhs;
    const int64_t kspan = L > 0 ? ((int64_t)(L - 1) * a.kts + D) * 2 : 0;
    const int64_t vspan = L > 0 ? ((int64_t)(L - 1) * a.vts + D) * 2 : 0;
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(kbase), (short)0, (int)(kspan < 0x7fffffff ? kspan : 0x7fffffff), 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(vbase), (short)0, (int)(vspan < 0x7fffffff ? vspan : 0x7fffffff), 0x00020000);
    const unsigned kts2 = (unsigned)(a.kts * 2), vts2 = (unsigned)(a.vts * 2);
    // Every cache byte is read once per step: loads carry the nontemporal (streaming) cache
    // policy, bit 1 of the buffer instruction's cache-policy operand ("nt"; 6% faster measured).
    constexpr int kStream = 2;
    // Tile offset of a tile past the split's end: every lane offset plus it lies in
    // [2^31, 2^32), outside any buffer (lane offsets stay below 2^31: 31 token strides at most).
    constexpr unsigned kSkip = 0x80000000u;
    // Loop-invariant lane offsets inside a tile: chunk idx = lane + 64 i is key idx / (D / 8),
    // 16-byte chunk idx % (D / 8), so 8 consecutive lanes read one 128-byte line.
    unsigned koff[VPL], voff[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int idx = lane + 64 * i;
        koff[i] = (unsigned)(idx / (D / 8)) * kts2 + (idx % (D / 8)) * 16;
        voff[i] = (unsigned)(idx / (D / 8)) * vts2 + (idx % (D / 8)) * 16;
    }

    f32x4 acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_i = kNegFloor, l_i = 0.f;

    struct TileRegs {
        s16x8 k[VPL];
        s16x8 v[VPL];
    };
    auto load_tile = [&](int t0, TileRegs& tr) {
        const unsigned kt = t0 < k1 ? (unsigned)t0 * kts2 : kSkip;
        const unsigned vt = t0 < k1 ? (unsigned)t0 * vts2 : kSkip;
#pragma unroll
        for (int i = 0; i < VPL; ++i)
            tr.k[i] = __builtin_bit_cast(s16x8, __builtin_amdgcn_raw_buffer_load_b128(krs, koff[i] + kt, 0, kStream));
#pragma unroll
        for (int i = 0; i < VPL; ++i)
            tr.v[i] = __builtin_bit_cast(s16x8, __builtin_amdgcn_raw_buffer_load_b128(vrs, voff[i] + vt, 0, kStream));
        // Keep tiles in issue order: the in-order load counter can then wait for the oldest
        // tile alone; a scheduler that interleaves two tiles' loads forces a full drain.
        __builtin_amdgcn_sched_barrier(0);
    };
    auto compute_tile = [&](int t0, const TileRegs& tr, int parity) {
        // Stage K and V in this wave's LDS (swizzled rows) for the operand reads.
        uint16_t* ks = klds[wave][parity % NPAR];
        uint16_t* vs = vlds[wave][parity % NPAR];
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int idx = lane + 64 * i;
            const int r = idx / (D / 8), ch = idx % (D / 8);
            *reinterpret_cast<s16x8*>(ks + r * D + ((ch ^ lds_swz<D>(r)) << 3)) = tr.k[i];
            *reinterpret_cast<s16x8*>(vs + r * D + ((ch ^ lds_swz<D>(r)) << 3)) = tr.v[i];
        }
        // S^T = K Q^T for the two 16-key blocks of the tile. Row rho of block kb is key
        // 8 (rho / 4) + 4 kb + rho % 4 (the order of the score registers); lane (rho, G) reads
        // d = 32 kk + 8 G .. + 7 of it (D = 16 pads d to 32 with zeros).
        f32x4 st[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            st[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
            const int key = 8 * (l16 >> 2) + 4 * kb + (l16 & 3);
#pragma unroll
            for (int kk = 0; kk < KD; ++kk) {
                const int d0 = 32 * kk + 8 * G;
                s16x8 kop = {0, 0, 0, 0, 0, 0, 0, 0};
                if (d0 < D) kop = *reinterpret_cast<const s16x8*>(ks + lds_off<D>(key, d0));
                st[kb] = T::mfma16(kop, qop[kk], st[kb]);
            }
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) st[kb] *= a.qk_scale;
        // Band mask, only on tiles that cross the band edge or the end of the cache.
        if (!(t0 >= rg.mid_lo && t0 + kTile <= rg.mid_hi)) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = t0 + 8 * G + 4 * kb + r;
                    const int rel = key - qi;
                    st[kb][r] = (rel >= lo_off && rel <= hi_off && key < L) ? st[kb][r] : -INFINITY;
                }
        }
        float mx = kNegFloor;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) mx = fmaxf(mx, st[kb][r]);
        // Row max across the 4 lane groups holding this row (lanes l16 + 16 G).
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = max_halves(mx);
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

    // NBUF tiles in registers: tile j computes while tiles j + 1 .. j + NBUF - 1 are in flight.
    const int nt = k1 > k0 ? (k1 - k0 + kTile - 1) / kTile : 0;
    TileRegs buf[NBUF];
#pragma unroll
    for (int i = 0; i < NBUF - 1; ++i) load_tile(k0 + i * kTile, buf[i]);
    for (int t = 0; t < nt; t += NBUF) {
#pragma unroll
        for (int i = 0; i < NBUF; ++i) {
            load_tile(k0 + (t + i + NBUF - 1) * kTile, buf[(i + NBUF - 1) % NBUF]);
            if (t + i < nt) compute_tile(k0 + (t + i) * kTile, buf[i], i & 1);
        }
    }

    // Row sum over the 4 lane groups (each summed its own keys); the max is already common.
    float l_row = l_i + __shfl_xor(l_i, 16);
    l_row = sum_halves(l_row);
    if (!row_ok) return;
    const bool empty = l_row == 0.f;
    const float inv = empty ? 0.f : 1.f / l_row;
    if (so.n == 1) {
        // Final output (flash_attn.py:147-154): lane writes d = 16 db + 4 G .. + 3 of its row.
        uint16_t* op = a.o + (int64_t)b * a.obs + (int64_t)qi * a.ots + (int64_t)h * a.ohs;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const int d0 = 16 * db + 4 * G;
            if (d0 < D) {
                u32x2 w = {T::pack2(acc[db][0] * inv, acc[db][1] * inv), T::pack2(acc[db][2] * inv, acc[db][3] * inv)};
                *reinterpret_cast<u32x2*>(op + d0) = w;
            }
        }
        if (G == 0) a.lse[(int64_t)h * a.lse_hs + (int64_t)b * a.nq + qi] = empty ? INFINITY : m_i + fast_log2(l_row);
    } else {
        // Normalized partial: O_s = o / l (16-bit), lse_s = m + log2(l) (-inf when empty).
        const int64_t prow = ((int64_t)(so.seg + split) * a.num_heads + h) * a.nq + qi;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const int d0 = 16 * db + 4 * G;
            if (d0 < D) {
                u32x2 w = {T::pack2(acc[db][0] * inv, acc[db][1] * inv), T::pack2(acc[db][2] * inv, acc[db][3] * inv)};
                *reinterpret_cast<u32x2*>(a.ws_o + prow * D + d0) = w;
            }
        }
        if (G == 0) a.ws_lse[prow] = empty ? -INFINITY : m_i + fast_log2(l_row);
    }
}

// Merge of one output row (batch, head, query) from the n split partials of its sequence,
// segments seg0 .. seg0 + n - 1: lse = log2(sum_s 2^lse_s), O = sum_s 2^(lse_s - lse) O_s.
// A wave merges R rows, each on its own GL = 64 / R lanes (the caller's lane / GL-th row). The
// splits go in chunks of up to GL (lane = split for the lse values; LPS lanes per partial O row,
// 8 elements each), and every load of a chunk is issued before the first is used, so a row
// costs one memory round trip per chunk; chunks after the first rescale the running sums to the
// new maximum. Reductions stay inside a row's lanes (xor offsets below GL).
template <int D, typename T, int R>
__device__ inline void merge_rows(const DecodeArgs& a, int b, int hh, int qq, int seg0, int n, int lane) {
    constexpr int GL = 64 / R;                          // lanes per row
    constexpr int LPS = D / 8;                          // lanes per split row (16 bytes each)
    static_assert(LPS <= GL, "a split row fits the row's lanes");
    constexpr int SPI = GL / LPS;                       // split rows per load of the row's lanes
    constexpr int CH = SPI * 16 < GL ? SPI * 16 : GL;   // splits per chunk (<= 16 loads per lane)
    constexpr int NL = CH / SPI;
    const int grp = lane / GL, gl = lane % GL;
    const int64_t rs = (int64_t)a.num_heads * a.nq;     // lse values between consecutive segments
    const int64_t row0 = ((int64_t)seg0 * a.num_heads + hh) * a.nq + qq;
    const float* lp = a.ws_lse + row0;
    const uint16_t* op = a.ws_o + row0 * D;
    const int sub = gl / LPS, d0 = (gl % LPS) * 8;
    float M = -INFINITY, lsum = 0.f;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int c0 = 0; c0 < n; c0 += CH) {
        const int cnt = n - c0 < CH ? n - c0 : CH;
        float ls = -INFINITY;
        if (gl < cnt) ls = lp[(int64_t)(c0 + gl) * rs];
        s16x8 ov[NL];
#pragma unroll
        for (int u = 0; u < NL; ++u) {
            const int sp = c0 + u * SPI + sub;
            ov[u] = s16x8{0, 0, 0, 0, 0, 0, 0, 0};
            if (sp < n) ov[u] = ld16(op + (int64_t)sp * rs * D + d0);
        }
        float mc = ls;
#pragma unroll
        for (int off = GL / 2; off >= 1; off >>= 1) mc = fmaxf(mc, __shfl_xor(mc, off));
        const float m_new = fmaxf(M, mc);
        if (m_new == -INFINITY) continue;
        const float sc = fast_exp2(M - m_new);
        const float w = fast_exp2(ls - m_new);
        float ws = w;
#pragma unroll
        for (int off = GL / 2; off >= 1; off >>= 1) ws += __shfl_xor(ws, off);
        lsum = lsum * sc + ws;
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] *= sc;
#pragma unroll
        for (int u = 0; u < NL; ++u) {
            const float wu = __shfl(w, grp * GL + u * SPI + sub);
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[c] += wu * T::to_float((uint16_t)ov[u][c]);
        }
        M = m_new;
    }
#pragma unroll
    for (int off = LPS; off < GL; off <<= 1)
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] += __shfl_xor(acc[c], off);
    const bool empty = M == -INFINITY;
    const float inv = empty ? 0.f : 1.f / lsum;
    if (gl < LPS) {
        uint16_t* out = a.o + (int64_t)b * a.obs + (int64_t)qq * a.ots + (int64_t)hh * a.ohs + gl * 8;
        u32x4 wv = {T::pack2(acc[0] * inv, acc[1] * inv), T::pack2(acc[2] * inv, acc[3] * inv),
                    T::pack2(acc[4] * inv, acc[5] * inv), T::pack2(acc[6] * inv, acc[7] * inv)};
        *reinterpret_cast<u32x4*>(out) = wv;
    }
    if (gl == 0) a.lse[(int64_t)hh * a.lse_hs + (int64_t)b * a.nq + qq] = empty ? INFINITY : M + fast_log2(lsum);
}

// R output rows per wave (R consecutive rows of one sequence, GROUP query heads x queries
// fastest), 64 / R lanes each; rows of a sequence of one split were written by the split-K pass.
template <int D, typename T, int R>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int64_t first = ((int64_t)blockIdx.x * 4 + wave) * R;  // over batch * num_heads * nq
    const int64_t total = (int64_t)a.batch * a.num_heads * a.nq;
    if (first >= total) return;
    const int b = (int)(first / ((int64_t)a.nq * a.num_heads));
    const int seg0 = a.seg_hdr[2 * b], n = a.seg_hdr[2 * b + 1];
    if (n <= 1) return;
    const int64_t row = first + lane / (64 / R);
    const int qq = (int)(row % a.nq);
    const int hh = (int)((row / a.nq) % a.num_heads);
    merge_rows<D, T, R>(a, b, hh, qq, seg0, n, lane);
}

// Split-K workgroups the current device holds at once: two per CU (64 KB of LDS each) up to
// head_dim 128, one at 256. The CU count is read once per device.
int resident_slots(int head_dim) {
    static int cus[64] = {};
    int dev = 0, n = 256;
    if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) {
        if (cus[dev] == 0) {
            int c = 0;
            if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
            cus[dev] = c;
        }
        n = cus[dev];
    }
    return n * (head_dim > 128 ? 1 : 2);
}

DecodeArgs make_args(const mykfa_decode_params& p, int splits, void* ws) {
    const mykfa_fwd_params& f = p.fwd;
    DecodeArgs a;
    a.n_new = p.seqlen_new;
    const bool append = p.k_new != nullptr && p.seqlen_new > 0;
    a.kn = append ? static_cast<const uint16_t*>(p.k_new) : nullptr;
    a.vn = append ? static_cast<const uint16_t*>(p.v_new) : nullptr;
    a.knbs = p.kn_batch_stride; a.knts = p.kn_token_stride; a.knhs = p.kn_head_stride;
    a.vnbs = p.vn_batch_stride; a.vnts = p.vn_token_stride; a.vnhs = p.vn_head_stride;
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
    a.units = f.num_kv_heads * a.row_tiles;
    a.num_heads = f.num_heads;
    a.batch = f.batch;
    a.nseg = splits > 1 ? splits * f.batch : f.batch;
    a.resident = resident_slots(f.head_dim) / ((a.units + kWaves - 1) / kWaves);
    const size_t seg_rows = (size_t)f.num_heads * f.max_seqlen_q;
    a.ws_o = splits > 1 ? static_cast<uint16_t*>(ws) : nullptr;
    a.ws_lse = splits > 1 ? reinterpret_cast<float*>(a.ws_o + (size_t)a.nseg * seg_rows * f.head_dim) : nullptr;
    a.seg_hdr = splits > 1 ? reinterpret_cast<int*>(a.ws_lse + (size_t)a.nseg * seg_rows) : nullptr;
    return a;
}

template <typename T>
hipError_t splitk_dtype(const DecodeArgs& a, int D, int num_kv_heads, hipStream_t s) {
    // Split slots: every sequence's splits are numbered in one running index (assign_split);
    // slots past the last split exit at once (they are dispatched last).
    dim3 grid(a.nseg, 1, (a.units + kWaves - 1) / kWaves);
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

template <typename T, int R>
hipError_t merge_rows_launch(const DecodeArgs& a, int D, hipStream_t s) {
    const int64_t rows = (int64_t)a.batch * a.num_heads * a.nq;
    dim3 grid((unsigned)((rows + 4 * R - 1) / (4 * R)));
    switch (D) {
        case 16: hipLaunchKernelGGL((decode_merge_kernel<16, T, R>), grid, dim3(256), 0, s, a); break;
        case 32: hipLaunchKernelGGL((decode_merge_kernel<32, T, R>), grid, dim3(256), 0, s, a); break;
        case 64: hipLaunchKernelGGL((decode_merge_kernel<64, T, R>), grid, dim3(256), 0, s, a); break;
        case 128: hipLaunchKernelGGL((decode_merge_kernel<128, T, R>), grid, dim3(256), 0, s, a); break;
        case 256:
            if constexpr (R <= 2) {
                hipLaunchKernelGGL((decode_merge_kernel<256, T, R>), grid, dim3(256), 0, s, a);
                break;
            }
            return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <typename T>
hipError_t merge_dtype(const DecodeArgs& a, int D, hipStream_t s) {
    // Four rows per wave (16 lanes each) when four divide a sequence's rows and a partial row
    // fits 16 lanes (D <= 128): a quarter of the workgroups for the same loads in flight. The
    // 4-query draft's merge measured 5.1 -> 3.7 us (85.8 against 87.1 us per layer); one query
    // unchanged (3.8 -> 3.7 us). Else one row per wave.
    const int64_t seq_rows = (int64_t)a.num_heads * a.nq;
    if (seq_rows % 4 == 0 && D <= 128) return merge_rows_launch<T, 4>(a, D, s);
    return merge_rows_launch<T, 1>(a, D, s);
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
    // Partial O and lse of num_splits segments per sequence on average, then the per-sequence
    // (first segment, split count) header the merge reads.
    return (size_t)num_splits * rows * ((size_t)head_dim * 2 + sizeof(float)) + (size_t)batch * 2 * sizeof(int);
}

int decode_default_splits(int batch, int num_heads, int num_kv_heads, int seqlen_q, int capacity) {
    // The slot pool (num_splits x batch segments): about 1400 keys of capacity per slot, since
    // each split costs a workgroup prologue and a partial row per query row that the merge reads
    // back, and longer splits stream longer runs of the cache (64 x 16K-cache batch, split-K +
    // merge with one split count for every sequence: 84.8 us at 12 splits of 1366 keys against
    // 86.3 at 46 of 352). Then at least ~512 workgroups (each kWaves KV-head units of one
    // sequence) for short batches and at least 128 keys per slot. The odd count avoids a multiple
    // of the 8 XCDs, which mattered when split s of every sequence sat at a fixed stride of the
    // grid; the device plan now sizes the splits from the actual lengths within this pool.
    const long long kvh = num_kv_heads > 0 ? num_kv_heads : 1;
    const long long group = num_heads > 0 ? (num_heads + kvh - 1) / kvh : 1;
    const long long rows = group * (seqlen_q > 0 ? seqlen_q : 1);
    const long long row_tiles = (rows + 15) / 16;
    const long long pairs = (long long)(batch > 0 ? batch : 1) * ((kvh * row_tiles + kWaves - 1) / kWaves);
    const long long cap = capacity > 0 ? capacity : 1;
    const long long chunk = 1408;
    long long splits = (cap + chunk - 1) / chunk;
    const long long fill = (512 + pairs - 1) / pairs;
    if (splits < fill) splits = fill;
    const long long max_by_len = (cap + 127) / 128;
    if (splits > max_by_len) splits = max_by_len;
    if (splits > 1023) splits = 1023;
    if (splits < 1) splits = 1;
    if (splits > 1 && splits % kXcds == 0) ++splits;
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

hipError_t decode_scratch(hipStream_t stream, void** ptr) {
    // Device addresses of `scratch`, one per GPU, resolved once per device: the device is the
    // one the launch stream belongs to (not necessarily the current one), made current while its
    // copy's address is taken.
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void* resolved[kMaxDevices] = {};
    int dev = 0;
    hipError_t e = hipStreamGetDevice(stream, &dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (resolved[dev] == nullptr) {
        int cur = 0;
        e = hipGetDevice(&cur);
        if (e != hipSuccess) return e;
        if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        const hipError_t back = cur != dev ? hipSetDevice(cur) : hipSuccess;
        if (e != hipSuccess) return e;
        if (back != hipSuccess) return back;
        if (p == nullptr) return hipErrorInvalidSymbol;
        resolved[dev] = p;
    }
    *ptr = resolved[dev];
    return hipSuccess;
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
