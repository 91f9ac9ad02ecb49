/*
 * TEST INFRASTRUCTURE ONLY -- CPU restatement of the reference's assignment
 * solver, used by tests/ as the checker and by bench.py as the CPU baseline.
 * The product path (mask_loss_amd) never links, loads or calls this file.
 *
 * Restates /root/reference/src/cpu/matching.cpp (AndyBarcia/mask_loss):
 *   big_from                     matching.cpp:71-83
 *   hungarian_assign (e-maxx)    matching.cpp:95-186
 *   greedy_assign_predictions    matching.cpp:193-229
 *   global_hungarian_assign      matching.cpp:239-286
 *   round_hungarian_assign       matching.cpp:294-366
 *   greedy_assign_all            matching.cpp:372-393
 *   pseudo_greedy_assign         matching.cpp:400-463
 *   assign_predictions_for_slice matching.cpp:476-571
 *   the at::parallel_for over L*B slices, matching.cpp:690-719
 *
 * Every floating-point operation on costs and potentials is done in double in
 * the same order as the reference (cur = (c - u[i0]) - v[j]; strict '<' for
 * both the minv update and the argmin, ascending j), so the outputs are the
 * reference's outputs bit for bit on the same double cost matrix.
 * Returns 0 on success, 1 if the solver finds no augmenting path (the
 * reference raises "Hungarian: no augmenting path found" there).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static double big_from(double x) {
    if (!isfinite(x) || x <= 0.0) return 1e15;
    double b = x * 0.5;
    if (!isfinite(b) || b < 1e6) b = 1e15;
    if (b > 1e290) b = 1e290;
    return b;
}

static int is_ok(double c, double inf_thresh) { return isfinite(c) && c < inf_thresh; }

/* rows = GT columns (cols[0..M)), columns = predictions preds[0..n). */
static int hungarian(const double* cost, const int64_t* preds, int64_t n,
                     const int64_t* cols, int64_t M, int64_t GT_out,
                     double inf_thresh, double BIG, int64_t* assign /* n */,
                     int64_t* iters_out) {
    for (int64_t k = 0; k < n; ++k) assign[k] = -1;
    if (M == 0 || n == 0 || n < M) return 0;
    double* u = (double*)calloc((size_t)(M + 1), sizeof(double));
    double* v = (double*)calloc((size_t)(n + 1), sizeof(double));
    int64_t* p = (int64_t*)calloc((size_t)(n + 1), sizeof(int64_t));
    int64_t* way = (int64_t*)calloc((size_t)(n + 1), sizeof(int64_t));
    double* minv = (double*)malloc((size_t)(n + 1) * sizeof(double));
    char* used = (char*)malloc((size_t)(n + 1));
    int rc = 0;
    int64_t iters = 0;
    for (int64_t i = 1; i <= M && rc == 0; ++i) {
        p[0] = i;
        int64_t j0 = 0;
        for (int64_t j = 0; j <= n; ++j) { minv[j] = INFINITY; used[j] = 0; }
        do {
            ++iters;
            used[j0] = 1;
            const int64_t i0 = p[j0];
            const int64_t col = cols[i0 - 1];
            double delta = INFINITY;
            int64_t j1 = 0;
            for (int64_t j = 1; j <= n; ++j) {
                if (used[j]) continue;
                const double raw = cost[preds[j - 1] * GT_out + col];
                const double cij = is_ok(raw, inf_thresh) ? raw : BIG;
                const double cur = cij - u[i0] - v[j];
                if (cur < minv[j]) { minv[j] = cur; way[j] = j0; }
                if (minv[j] < delta) { delta = minv[j]; j1 = j; }
            }
            if (!isfinite(delta)) { rc = 1; break; }
            for (int64_t j = 0; j <= n; ++j) {
                if (used[j]) { u[p[j]] += delta; v[j] -= delta; }
                else minv[j] -= delta;
            }
            j0 = j1;
        } while (p[j0] != 0);
        if (rc) break;
        do { const int64_t j1 = way[j0]; p[j0] = p[j1]; j0 = j1; } while (j0 != 0);
    }
    if (rc == 0) {
        for (int64_t j = 1; j <= n; ++j)
            if (p[j] > 0) assign[j - 1] = p[j] - 1;
    }
    if (iters_out) *iters_out += iters;
    free(u); free(v); free(p); free(way); free(minv); free(used);
    return rc;
}

static void greedy_preds(const double* cost, const int64_t* preds, int64_t npreds,
                         const int64_t* valid, int64_t nvalid, double inf_thresh,
                         int64_t* cap, int64_t GT_out, int64_t* p2g) {
    for (int64_t idx = 0; idx < npreds; ++idx) {
        const int64_t q = preds[idx];
        if (p2g[q] >= 0) continue;
        double best = INFINITY;
        int64_t bg = -1;
        for (int64_t t = 0; t < nvalid; ++t) {
            const int64_t a = valid[t];
            if (cap[a] <= 0) continue;
            const double c = cost[q * GT_out + a];
            if (!is_ok(c, inf_thresh)) continue;
            if (c < best) { best = c; bg = a; }
        }
        if (bg >= 0) { p2g[q] = bg; if (cap[bg] > 0) cap[bg] -= 1; }
    }
}

/* strategy: 0 global, 1 round, 2 greedy, 3 pseudo-greedy (matching.cpp:60-65) */
int ml_oracle_assign_slice(const double* cost, int64_t Q, int64_t GT_out,
                           double inf_thresh, int64_t topk, int strategy,
                           int64_t* pred_to_gt, int64_t* pred_round,
                           int64_t* iters) {
    for (int64_t q = 0; q < Q; ++q) { pred_to_gt[q] = -1; pred_round[q] = -1; }
    if (Q == 0 || GT_out == 0 || topk == 0) return 0;
    int rc = 0;
    int64_t* valid = (int64_t*)malloc((size_t)GT_out * sizeof(int64_t));
    int64_t nvalid = 0;
    for (int64_t g = 0; g < GT_out; ++g) {
        for (int64_t q = 0; q < Q; ++q)
            if (is_ok(cost[q * GT_out + g], inf_thresh)) { valid[nvalid++] = g; break; }
    }
    int64_t* all = (int64_t*)malloc((size_t)Q * sizeof(int64_t));
    for (int64_t q = 0; q < Q; ++q) all[q] = q;
    int64_t* asg = (int64_t*)malloc((size_t)Q * sizeof(int64_t));
    int64_t* cap = (int64_t*)calloc((size_t)GT_out, sizeof(int64_t));
    const int64_t ncol_cap = nvalid * (topk > 0 ? topk : 0) + 1;
    int64_t* cols = (int64_t*)malloc((size_t)(ncol_cap < Q + 1 ? Q + 1 : ncol_cap) * sizeof(int64_t));
    if (nvalid > 0 && topk > 0) {
        const double BIG = big_from(inf_thresh);
        if (strategy == 0) {
            int64_t M = 0;
            for (int64_t rep = 0; rep < topk && M < Q; ++rep)
                for (int64_t t = 0; t < nvalid; ++t) {
                    cols[M++] = valid[t];
                    if (M >= Q) break;
                }
            if (M > 0) {
                rc = hungarian(cost, all, Q, cols, M, GT_out, inf_thresh, BIG, asg, iters);
                if (!rc)
                    for (int64_t k = 0; k < Q; ++k) {
                        if (asg[k] < 0) continue;
                        const int64_t a = cols[asg[k]];
                        if (!is_ok(cost[k * GT_out + a], inf_thresh)) continue;
                        pred_to_gt[k] = a;
                    }
            }
        } else if (strategy == 1) {
            for (int64_t t = 0; t < nvalid; ++t) cap[valid[t]] = topk;
            int64_t nrem = Q;
            int64_t* rem = (int64_t*)malloc((size_t)Q * sizeof(int64_t));
            int64_t* nxt = (int64_t*)malloc((size_t)Q * sizeof(int64_t));
            for (int64_t q = 0; q < Q; ++q) rem[q] = q;
            for (int64_t r = 0; r < topk && rc == 0; ++r) {
                int64_t M = 0;
                for (int64_t t = 0; t < nvalid; ++t)
                    if (cap[valid[t]] > 0) cols[M++] = valid[t];
                if (M == 0 || nrem == 0) break;
                if (M > nrem) M = nrem;
                if (M == 0) break;
                rc = hungarian(cost, rem, nrem, cols, M, GT_out, inf_thresh, BIG, asg, iters);
                if (rc) break;
                int64_t nn = 0;
                for (int64_t k = 0; k < nrem; ++k) {
                    const int64_t q = rem[k];
                    if (asg[k] >= 0) {
                        const int64_t a = cols[asg[k]];
                        if (!is_ok(cost[q * GT_out + a], inf_thresh)) { nxt[nn++] = q; continue; }
                        pred_to_gt[q] = a;
                        if (cap[a] > 0) cap[a] -= 1;
                    } else nxt[nn++] = q;
                }
                memcpy(rem, nxt, (size_t)nn * sizeof(int64_t));
                nrem = nn;
                if (nrem == 0) break;
            }
            free(rem); free(nxt);
        } else if (strategy == 2) {
            for (int64_t t = 0; t < nvalid; ++t) cap[valid[t]] = topk;
            greedy_preds(cost, all, Q, valid, nvalid, inf_thresh, cap, GT_out, pred_to_gt);
        } else if (strategy == 3) {
            for (int64_t t = 0; t < nvalid; ++t) cap[valid[t]] = topk;
            int64_t M = 0;
            for (int64_t t = 0; t < nvalid; ++t) { cols[M++] = valid[t]; if (M >= Q) break; }
            if (M > 0) {
                rc = hungarian(cost, all, Q, cols, M, GT_out, inf_thresh, BIG, asg, iters);
                if (!rc)
                    for (int64_t k = 0; k < Q; ++k) {
                        if (asg[k] < 0) continue;
                        const int64_t a = cols[asg[k]];
                        if (!is_ok(cost[k * GT_out + a], inf_thresh)) continue;
                        pred_to_gt[k] = a;
                        if (cap[a] > 0) cap[a] -= 1;
                    }
            }
            if (!rc) {
                int64_t nr = 0;
                for (int64_t q = 0; q < Q; ++q) if (pred_to_gt[q] < 0) all[nr++] = q;
                if (nr > 0) greedy_preds(cost, all, nr, valid, nvalid, inf_thresh, cap, GT_out, pred_to_gt);
            }
        } else {
            rc = 2;
        }
    }
    if (rc == 0) {
        /* rank matched predictions per GT by (cost, q); matching.cpp:533-565 */
        for (int64_t q = 0; q < Q; ++q) {
            const int64_t g = pred_to_gt[q];
            if (g < 0 || g >= GT_out) continue;
            if (!is_ok(cost[q * GT_out + g], inf_thresh)) pred_to_gt[q] = -1;
        }
        for (int64_t g = 0; g < GT_out; ++g) {
            int64_t r = 0;
            /* selection by (cost, q) ascending without allocation: repeat min search */
            for (;;) {
                if (r >= topk) break;
                int64_t best = -1;
                double bc = 0.0;
                for (int64_t q = 0; q < Q; ++q) {
                    if (pred_to_gt[q] != g || pred_round[q] >= 0) continue;
                    const double c = cost[q * GT_out + g];
                    if (best < 0 || c < bc) { best = q; bc = c; }
                }
                if (best < 0) break;
                pred_round[best] = r++;
            }
        }
    }
    free(valid); free(all); free(asg); free(cap); free(cols);
    return rc;
}

/* N independent (Q x GT_out) slices; slice t written to p2g/pr + t*Q.
 * nthreads > 1 splits slices over OpenMP threads (grain 1), as the reference
 * splits them over at::parallel_for (matching.cpp:690). */
int ml_oracle_assign_batch(const double* costs, int64_t N, int64_t Q, int64_t GT_out,
                           double inf_thresh, int64_t topk, int strategy,
                           int64_t* p2g, int64_t* pr, int nthreads,
                           int64_t* iters_per_slice) {
    int rc_all = 0;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads > 0 ? nthreads : 1) reduction(|:rc_all)
#endif
    for (int64_t t = 0; t < N; ++t) {
        int64_t it = 0;
        rc_all |= ml_oracle_assign_slice(costs + t * Q * GT_out, Q, GT_out, inf_thresh, topk,
                                         strategy, p2g + t * Q, pr + t * Q, &it);
        if (iters_per_slice) iters_per_slice[t] = it;
    }
    (void)nthreads;
    return rc_all;
}
