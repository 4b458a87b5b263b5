/*
 * ORACLE -- test infrastructure only, never product code.
 *
 * Independent float64 restatement of the per-query-row attention math of the
 * reference's scalar kernel (metal_flash_attn/_kernel.py:32-87, `flash_attn_fwd`):
 *   center = i + (Lk - Lq)                                   (:59)
 *   kmax   = causal ? center + 1 : Lk; kmax = min(kmax, center + wr + 1) if wr >= 0
 *   kmin   = wl >= 0 ? max(0, center - wl) : 0                (:60-62)
 *   s      = scale * q.k                                     (:73-75)
 *   s      = softcap * tanh(s / softcap)       if softcap > 0 (:76)
 *   s     -= slope[b*Hq + h] * |center - j|    if ALiBi       (:77)
 *   O      = sum_j softmax(s)_j v_j, or 0 when no key is valid (:78-86)
 *   hkv    = h / (Hq / Hkv)                                  (:54)
 * Written as a two-pass (max, then exp-sum) evaluation in double precision,
 * i.e. a different evaluation order from both the reference's online
 * softmax and its chunked torch path, so that it can pin them.
 *
 * Layout: heads-second, contiguous: q [B,Hq,Lq,D], k/v [B,Hkv,Lk,D],
 * o [B,Hq,Lq,D] (double).  alibi: [B*Hq] or NULL.  lse: [B,Hq,Lq] (double)
 * or NULL; when given, it receives m + log(l), the log of the softmax
 * normaliser (-inf for a row with no valid key), which the reference
 * computes but never returns.
 */
#include <math.h>
#include <stdlib.h>

int oracle_stream_fwd(const float* q, const float* k, const float* v, double* o,
                      int B, int Hq, int Hkv, int Lq, int Lk, int D,
                      int causal, double scale, double softcap, int wl, int wr,
                      const float* alibi, double* lse)
{
    if (Hkv <= 0 || Hq % Hkv != 0) return -1;
    double* s = (double*)malloc(sizeof(double) * (Lk > 0 ? Lk : 1));
    if (!s) return -2;
    const int group = Hq / Hkv;
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < Hq; ++h) {
            const int hk = h / group;
            const float* kb = k + ((size_t)(b * Hkv + hk) * Lk) * D;
            const float* vb = v + ((size_t)(b * Hkv + hk) * Lk) * D;
            const double slope = alibi ? (double)alibi[b * Hq + h] : 0.0;
            for (int i = 0; i < Lq; ++i) {
                const float* qi = q + ((size_t)(b * Hq + h) * Lq + i) * D;
                double* oi = o + ((size_t)(b * Hq + h) * Lq + i) * D;
                const long center = (long)i + (long)Lk - (long)Lq;
                long kmax = causal ? center + 1 : Lk;
                if (wr >= 0 && center + wr + 1 < kmax) kmax = center + wr + 1;
                if (kmax > Lk) kmax = Lk;
                long kmin = 0;
                if (wl >= 0 && center - wl > 0) kmin = center - wl;
                for (int d = 0; d < D; ++d) oi[d] = 0.0;
                if (lse) lse[(size_t)(b * Hq + h) * Lq + i] = -INFINITY;
                if (kmin >= kmax) continue;
                double m = -INFINITY;
                for (long j = kmin; j < kmax; ++j) {
                    double acc = 0.0;
                    const float* kj = kb + (size_t)j * D;
                    for (int d = 0; d < D; ++d) acc += (double)qi[d] * (double)kj[d];
                    acc *= scale;
                    if (softcap > 0.0) acc = softcap * tanh(acc / softcap);
                    if (alibi) acc -= slope * fabs((double)(center - j));
                    s[j] = acc;
                    if (acc > m) m = acc;
                }
                double l = 0.0;
                for (long j = kmin; j < kmax; ++j) {
                    const double p = exp(s[j] - m);
                    l += p;
                    const float* vj = vb + (size_t)j * D;
                    for (int d = 0; d < D; ++d) oi[d] += p * (double)vj[d];
                }
                for (int d = 0; d < D; ++d) oi[d] /= l;
                if (lse) lse[(size_t)(b * Hq + h) * Lq + i] = m + log(l);
            }
        }
    free(s);
    return 0;
}
