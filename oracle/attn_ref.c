/*
 * Float64 brute-force attention, forward and backward — TEST INFRASTRUCTURE ONLY.
 *
 * An independent, loop-by-loop statement of the mathematics the reference's path computes,
 * used to pin the torch oracle (oracle/attention.py); never linked into the product.
 *   mask    : query i sees key j iff i + Lk - Lq - wl <= j <= i + Lk - Lq + wr, 0 <= j < Lk
 *             (flash_attn.py:14-18; wl/wr already resolved by _window, flash_attn.py:435-439)
 *   forward : s_j = scale * q_i . k_j, P = softmax(s), o_i = sum_j P_j v_j,
 *             lse2_i = log2(sum_j exp(s_j)); rows with no visible key: o = 0, lse2 = +inf
 *             (flash_attn.py:147-153)
 *   backward: dP_j = do_i . v_j, D_i = sum_j P_j dP_j (= do_i . o_i, flash_attn.py:215),
 *             dS_j = P_j (dP_j - D_i), dq_i = scale sum_j dS_j k_j,
 *             dk_j += scale dS_j q_i, dv_j += P_j do_i; GQA heads h map to kv head h / group
 *             and their dk/dv contributions are summed (flash_attn.py:300-311).
 * Layouts: q/o/do/dq (B, Lq, H, D), k/v/dk/dv (B, Lk, Hkv, D), lse2 (H, B * Lq), all dense.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

static int visible(long long i, long long j, long long lq, long long lk, long long wl, long long wr) {
    long long pos = i + lk - lq;
    return j >= 0 && j < lk && j >= pos - wl && j <= pos + wr;
}

int attn_ref(int B, int Lq, int Lk, int H, int Hkv, int D, int wl, int wr, double scale,
             const double* q, const double* k, const double* v, const double* dout,
             double* o, double* lse2, double* dq, double* dk, double* dv) {
    if (B < 0 || Lq < 0 || Lk < 0 || H <= 0 || Hkv <= 0 || D <= 0 || H % Hkv) return 1;
    const int group = H / Hkv;
    double* s = (double*)malloc(sizeof(double) * (Lk > 0 ? Lk : 1));
    double* p = (double*)malloc(sizeof(double) * (Lk > 0 ? Lk : 1));
    double* dp = (double*)malloc(sizeof(double) * (Lk > 0 ? Lk : 1));
    if (!s || !p || !dp) return 2;
    if (dk) memset(dk, 0, sizeof(double) * (size_t)B * Lk * Hkv * D);
    if (dv) memset(dv, 0, sizeof(double) * (size_t)B * Lk * Hkv * D);
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h) {
            const int kh = h / group;
            for (int i = 0; i < Lq; ++i) {
                const double* qi = q + (((size_t)b * Lq + i) * H + h) * D;
                double m = -INFINITY;
                int any = 0;
                for (int j = 0; j < Lk; ++j) {
                    if (!visible(i, j, Lq, Lk, wl, wr)) continue;
                    const double* kj = k + (((size_t)b * Lk + j) * Hkv + kh) * D;
                    double acc = 0;
                    for (int d = 0; d < D; ++d) acc += qi[d] * kj[d];
                    s[j] = acc * scale;
                    if (s[j] > m) m = s[j];
                    any = 1;
                }
                double l = 0;
                for (int j = 0; j < Lk; ++j) {
                    p[j] = 0;
                    if (any && visible(i, j, Lq, Lk, wl, wr)) {
                        p[j] = exp(s[j] - m);
                        l += p[j];
                    }
                }
                double* oi = o + (((size_t)b * Lq + i) * H + h) * D;
                for (int d = 0; d < D; ++d) oi[d] = 0;
                if (any) {
                    for (int j = 0; j < Lk; ++j) p[j] /= l;
                    for (int j = 0; j < Lk; ++j) {
                        if (p[j] == 0) continue;
                        const double* vj = v + (((size_t)b * Lk + j) * Hkv + kh) * D;
                        for (int d = 0; d < D; ++d) oi[d] += p[j] * vj[d];
                    }
                    lse2[(size_t)h * B * Lq + (size_t)b * Lq + i] = (m + log(l)) / log(2.0);
                } else {
                    lse2[(size_t)h * B * Lq + (size_t)b * Lq + i] = INFINITY;
                }
                if (!dout) continue;
                const double* doi = dout + (((size_t)b * Lq + i) * H + h) * D;
                double* dqi = dq + (((size_t)b * Lq + i) * H + h) * D;
                for (int d = 0; d < D; ++d) dqi[d] = 0;
                if (!any) continue;
                double Di = 0;
                for (int j = 0; j < Lk; ++j) {
                    dp[j] = 0;
                    if (!visible(i, j, Lq, Lk, wl, wr)) continue;
                    const double* vj = v + (((size_t)b * Lk + j) * Hkv + kh) * D;
                    double acc = 0;
                    for (int d = 0; d < D; ++d) acc += doi[d] * vj[d];
                    dp[j] = acc;
                    Di += p[j] * acc;
                }
                for (int j = 0; j < Lk; ++j) {
                    if (!visible(i, j, Lq, Lk, wl, wr)) continue;
                    const double ds = p[j] * (dp[j] - Di);
                    const double* kj = k + (((size_t)b * Lk + j) * Hkv + kh) * D;
                    double* dkj = dk + (((size_t)b * Lk + j) * Hkv + kh) * D;
                    double* dvj = dv + (((size_t)b * Lk + j) * Hkv + kh) * D;
                    for (int d = 0; d < D; ++d) {
                        dqi[d] += scale * ds * kj[d];
                        dkj[d] += scale * ds * qi[d];
                        dvj[d] += p[j] * doi[d];
                    }
                }
            }
        }
    free(s);
    free(p);
    free(dp);
    return 0;
}
