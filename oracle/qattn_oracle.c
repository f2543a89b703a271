/*
 * qattn_oracle.c -- CPU restatement of the reference's tree-verify attention.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product path (qattention_amd/,
 * src/) may link, load or call this file.  It is built by oracle/build.py into
 * oracle/_build/libqattn_oracle.so and used by tests/, by
 * __graft_entry__.smoke() as the checker, and by bench.py's cpu_baseline leg.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the saifmb0/QAttention tree).  The checks that pin each
 * function (known answers, invariants, library special cases, planted
 * mistakes) live in tests/test_oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Number of nodes of a complete b-ary tree of depth d.
 * Follows src/tree_mask.py:78-83 (b == 1 gives d + 1). */
int64_t oracle_num_tree_nodes(int b, int d) {
    if (b < 1 || d < 0) return -1;
    if (b == 1) return (int64_t)d + 1;
    int64_t p = 1;
    for (int i = 0; i < d + 1; ++i) {
        p *= b;
        if (p > ((int64_t)1 << 40)) return -1;
    }
    return (p - 1) / (b - 1);
}

/* BFS parent array of a complete b-ary tree, root parent = -1.
 * Follows src/tree_mask.py:86-113: children are appended frontier by
 * frontier, b per node, in order.  Returns N, or -1 if cap is too small. */
int64_t oracle_build_tree(int b, int d, int32_t *parent, int64_t cap) {
    int64_t n = oracle_num_tree_nodes(b, d);
    if (n < 0 || n > cap) return -1;
    int64_t len = 0;
    parent[len++] = -1;
    int64_t f_lo = 0, f_hi = 1; /* current frontier = [f_lo, f_hi) */
    for (int lvl = 0; lvl < d; ++lvl) {
        int64_t next_lo = len;
        for (int64_t node = f_lo; node < f_hi; ++node)
            for (int c = 0; c < b; ++c) parent[len++] = (int32_t)node;
        f_lo = next_lo;
        f_hi = len;
    }
    return len;
}

/* Ancestor walk of the heap-indexed kernel, one row per packed token.
 * Follows src/ragged_attn.py:323-324 (cur = q, prev = -1), :340 (attend iff
 * cur != prev), :376-377 (prev = cur; cur = max(cur - 1, 0) // b, clamp
 * before the divide) for MAX_DEPTH + 1 steps (:338).  out[t*(S+1) + s] holds
 * the sequence-local ancestor attended at step s, or -1 when step s is a
 * repeat.  cu is the [B+1] prefix-sum of sequence lengths. */
void oracle_ancestor_table_heap(const int32_t *cu, int B, int b, int max_depth,
                                int32_t *out) {
    const int S1 = max_depth + 1;
    for (int seq = 0; seq < B; ++seq) {
        const int32_t n = cu[seq + 1] - cu[seq];
        for (int32_t q = 0; q < n; ++q) {
            int32_t *row = out + (int64_t)(cu[seq] + q) * S1;
            int32_t cur = q, prev = -1;
            for (int s = 0; s < S1; ++s) {
                row[s] = (cur != prev) ? cur : -1;
                prev = cur;
                int32_t m = cur - 1 > 0 ? cur - 1 : 0;
                cur = m / b;
            }
        }
    }
}

/* Ancestor walk of the explicit-parent kernel.
 * Follows src/ragged_attn.py:650-698: cur = q, prev = -1; attend iff
 * cur != prev; cur = parents[seq_start + cur].  A root must self-loop
 * (parents[root] == root, :613).  The reference leaves an out-of-range parent
 * undefined (it reads outside the sequence); this restatement, like the HIP
 * kernel, stops the walk there (treated as a self-loop). */
void oracle_ancestor_table_parents(const int32_t *cu, int B, const int32_t *parents,
                                   int max_depth, int32_t *out) {
    const int S1 = max_depth + 1;
    for (int seq = 0; seq < B; ++seq) {
        const int32_t start = cu[seq], n = cu[seq + 1] - cu[seq];
        for (int32_t q = 0; q < n; ++q) {
            int32_t *row = out + (int64_t)(start + q) * S1;
            int32_t cur = q, prev = -1;
            for (int s = 0; s < S1; ++s) {
                row[s] = (cur != prev) ? cur : -1;
                prev = cur;
                int32_t p = parents[start + cur];
                cur = (p >= 0 && p < n) ? p : cur;
            }
        }
    }
}

/* Sparse ancestor attention in double precision.
 *
 * For each packed token t (sequence seq, local index via cu) and query head h:
 *   keys  = { prefix rows 0..L-1 of seq (all attended, src/ragged_attn.py:1764-1798) }
 *         U { tree rows cu[seq] + anc[t][s] for every s with anc >= 0 (:338-377) }
 *   s_a   = scale * <q[t,h,:], k[a, kvh, :]>
 *   o     = sum_a exp(s_a - m) v_a / sum_a exp(s_a - m)      (:359-381)
 *   lse   = m + log(sum_a exp(s_a - m))                          (:484-488)
 * kvh = h / (Hq / Hkv) reproduces repeat_kv (scripts/e2e_benchmark.py:1581);
 * Hkv == Hq is the reference layout.
 *
 * Layouts (contiguous, float32 inputs):
 *   q  [T][Hq][D],  k/v  [T][Hkv][D],  anc [T][S1]
 *   kp/vp (optional, L > 0) [B][L][Hkv][D]
 *   o  [T][Hq][D] double,  lse [T][Hq] double (optional)
 * Tokens are independent, so an OpenMP build spreads them over threads; each
 * output is still summed in the same order by one thread (deterministic). */
void oracle_tree_attn(const float *q, const float *k, const float *v,
                      const int32_t *cu, int B, int Hq, int Hkv, int D,
                      const int32_t *anc, int S1,
                      const float *kp, const float *vp, int L,
                      double scale, double *o, double *lse) {
    const int g = Hq / Hkv;
    if (B <= 0) return;
    /* tokens [cu[0], cu[B]); rows outside every sequence are left untouched */
    const int32_t t_lo = cu[0], t_hi = cu[B];
#pragma omp parallel
    {
        double *scores = (double *)malloc(sizeof(double) * (size_t)(L + S1));
        int64_t *rows = (int64_t *)malloc(sizeof(int64_t) * (size_t)(L + S1));
#pragma omp for schedule(dynamic, 64)
        for (int32_t t = t_lo; t < t_hi; ++t) {
            /* sequence of token t: the last seq with cu[seq] <= t (cu is
             * non-decreasing, so cu[seq + 1] > t) */
            int lo = 0, hi = B - 1;
            while (lo < hi) {
                int mid = (lo + hi + 1) / 2;
                if (cu[mid] <= t) lo = mid; else hi = mid - 1;
            }
            const int seq = lo;
            for (int h = 0; h < Hq; ++h) {
                const int kvh = h / g;
                const float *qr = q + ((int64_t)t * Hq + h) * D;
                int nk = 0;
                double m = -INFINITY;
                /* prefix keys */
                for (int j = 0; j < L; ++j) {
                    const float *kr = kp + (((int64_t)seq * L + j) * Hkv + kvh) * D;
                    double s = 0.0;
                    for (int d = 0; d < D; ++d) s += (double)qr[d] * (double)kr[d];
                    s *= scale;
                    scores[nk] = s;
                    rows[nk] = -1 - (int64_t)j; /* negative: prefix row j */
                    ++nk;
                    if (s > m) m = s;
                }
                /* tree ancestors */
                for (int s1 = 0; s1 < S1; ++s1) {
                    int32_t a = anc[(int64_t)t * S1 + s1];
                    if (a < 0) continue;
                    int64_t row = (int64_t)cu[seq] + a;
                    const float *kr = k + (row * Hkv + kvh) * D;
                    double s = 0.0;
                    for (int d = 0; d < D; ++d) s += (double)qr[d] * (double)kr[d];
                    s *= scale;
                    scores[nk] = s;
                    rows[nk] = row;
                    ++nk;
                    if (s > m) m = s;
                }
                double *orow = o + ((int64_t)t * Hq + h) * D;
                for (int d = 0; d < D; ++d) orow[d] = 0.0;
                double l = 0.0;
                for (int i = 0; i < nk; ++i) {
                    double p = exp(scores[i] - m);
                    l += p;
                    const float *vr;
                    if (rows[i] < 0) {
                        int64_t j = -1 - rows[i];
                        vr = vp + (((int64_t)seq * L + j) * Hkv + kvh) * D;
                    } else {
                        vr = v + (rows[i] * Hkv + kvh) * D;
                    }
                    for (int d = 0; d < D; ++d) orow[d] += p * (double)vr[d];
                }
                /* l == 0 cannot happen for a valid token (step 0 always
                 * attends itself); keep the reference's guard (:379-380). */
                double l_safe = (l == 0.0) ? 1.0 : l;
                for (int d = 0; d < D; ++d) orow[d] /= l_safe;
                if (lse) lse[(int64_t)t * Hq + h] = m + log(l_safe);
            }
        }
        free(scores);
        free(rows);
    }
}

/* Two-state softmax merge, double precision.
 * Follows src/ragged_attn.py:1599-1616:
 *   mx = max(lse_p, lse_t); w_p = exp(lse_p - mx); w_t = exp(lse_t - mx)
 *   out = (w_p o_p + w_t o_t) / max(w_p + w_t, 1e-8)
 * All arrays contiguous: lse [n_pos], o [n_pos][D]. */
void oracle_lse_merge(const float *lse_p, const float *lse_t, const float *o_p,
                      const float *o_t, int64_t n_pos, int D, double *out) {
    for (int64_t i = 0; i < n_pos; ++i) {
        double a = lse_p[i], b = lse_t[i];
        double mx = a > b ? a : b;
        double wp = exp(a - mx), wt = exp(b - mx);
        double ws = wp + wt;
        if (ws < 1e-8) ws = 1e-8;
        for (int d = 0; d < D; ++d)
            out[i * D + d] = (wp * (double)o_p[i * D + d] + wt * (double)o_t[i * D + d]) / ws;
    }
}
