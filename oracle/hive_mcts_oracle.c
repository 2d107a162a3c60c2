/*
 * hive_mcts_oracle.c -- CPU restatement of the reference's MCTS tree kernels
 * (hive_gpu/csrc/mcts_tree.cuh) under the canonical order of effect:
 * simulations run one after another in simulation-index order, so each
 * selection sees the virtual losses of earlier ones, the earliest
 * simulation reaching an unexpanded leaf expands it, node ids are handed
 * out in that order and float updates happen in that order.
 *
 * TEST INFRASTRUCTURE ONLY (see hive_oracle.c).  Pinned by the invariants in
 * tests/test_oracle_mcts.py (virtual losses undone, visit-count
 * conservation, child contiguity and order, sign alternation, pool
 * exhaustion, terminal values) and by hand-built trees with known PUCT
 * choices.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "hive_oracle.h"

enum { DEPTH = 128 };

static inline int64_t at(const or_tree* t, int64_t g, int node) { return g * t->M + node; }

/* puct_score mcts_tree.cuh:55-67 */
static float puct(const or_tree* t, int64_t parent, int64_t child, float c_puct) {
    int n = t->vc[child];
    float q = n > 0 ? (-t->tv[child] / (float)n) : 0.0f;
    q -= t->vq[child];
    float e = c_puct * t->pr[child] * sqrtf((float)t->vc[parent]) / (1.0f + (float)n);
    return q + e;
}

/* deterministic_completed_q_child mcts_tree.cuh:77-143 */
static float child_q(const or_tree* t, int64_t ci) {
    float visits = (float)t->vc[ci];
    float q = visits > 0.0f ? (-t->tv[ci] / visits) : t->ciq[ci];
    return q - t->vq[ci];
}

static int completed_q_child(const or_tree* t, int64_t g, int first, int count, float sigma) {
    float sum_visits = 0.0f, mx = -1e30f, se = 0.0f;
    int lim = count;
    for (int c = 0; c < count; c++)
        if (first + c < 0 || first + c >= t->M) { lim = c; break; }
    for (int c = 0; c < lim; c++) sum_visits += (float)t->vc[at(t, g, first + c)];
    for (int c = 0; c < lim; c++) {
        int64_t ci = at(t, g, first + c);
        float lq = logf(fmaxf(t->pr[ci], 1e-20f)) + sigma * child_q(t, ci);
        if (lq > mx) mx = lq;
    }
    for (int c = 0; c < lim; c++) {
        int64_t ci = at(t, g, first + c);
        se += expf(logf(fmaxf(t->pr[ci], 1e-20f)) + sigma * child_q(t, ci) - mx);
    }
    se = fmaxf(se, 1e-20f);
    int best = -1;
    float bs = -1e30f, denom = 1.0f + sum_visits;
    for (int c = 0; c < lim; c++) {
        int64_t ci = at(t, g, first + c);
        float visits = (float)t->vc[ci];
        float pi0 = expf(logf(fmaxf(t->pr[ci], 1e-20f)) + sigma * child_q(t, ci) - mx) / se;
        float score = pi0 - (visits / denom);
        if (score > bs) { bs = score; best = first + c; }
    }
    return best;
}

typedef struct {
    int32_t* leaf;
    uint8_t* paths;
    int32_t* plen;
    int32_t* vl;
    int32_t* vlen;
} sel_out;

static void blank(const sel_out* o, int64_t s) { o->leaf[s] = -1; o->plen[s] = 0; o->vlen[s] = 0; }

static void record_move(const or_tree* t, const sel_out* o, int64_t s, int64_t ni, int* plen) {
    if (*plen < DEPTH) {
        memcpy(o->paths + (s * DEPTH + *plen) * 6, t->mb + ni * 6, 6);
        (*plen)++;
    }
}

static void take_child(const or_tree* t, const sel_out* o, int64_t s, int64_t g, int node, int det, float qp,
                       int* plen, int* vlen) {
    int64_t ni = at(t, g, node);
    t->vc[ni] += 1;
    if (det) t->vq[ni] += qp;
    else t->tv[ni] += -1.0f;
    if (*vlen < DEPTH) o->vl[s * DEPTH + (*vlen)++] = node;
    record_move(t, o, s, ni, plen);
}

/* best child by PUCT, first maximum, scores must exceed -1e30 */
static int puct_argmax(const or_tree* t, int64_t g, int node, int first, int count, float c_puct,
                       const int8_t* alive, int max_root) {
    int best = -1;
    float bs = -1e30f;
    for (int c = 0; c < count; c++) {
        int child = first + c;
        if (child < 0 || child >= t->M) break;
        if (alive && (c >= max_root || !alive[c])) continue;
        float sc = puct(t, at(t, g, node), at(t, g, child), c_puct);
        if (sc > bs) { bs = sc; best = child; }
    }
    return best;
}

static int descend(const or_tree* t, const sel_out* o, int64_t s, int64_t g, int node, int from_iter, float c_puct,
                   int det, float sigma, float qp, int* plen, int* vlen) {
    for (int it = from_iter; it < DEPTH; it++) {
        int64_t ni = at(t, g, node);
        int f = t->fc[ni], n = t->nc[ni];
        if (f < 0 || t->it[ni] || n == 0 || n <= 0 || n > 1024) break;
        int best = det ? completed_q_child(t, g, f, n, sigma) : puct_argmax(t, g, node, f, n, c_puct, NULL, 0);
        if (best < 0) break;
        node = best;
        take_child(t, o, s, g, node, det, qp, plen, vlen);
    }
    return node;
}

/* mcts_select_with_root_slots_kernel mcts_tree.cuh:811-955 */
void or_mcts_select_slots(const or_tree* t, const int8_t* active, const int32_t* roots, const int32_t* slots, int C,
                          int max_root, float c_puct, int64_t B, int W, int det, float sigma, float qp,
                          int32_t* leaf, uint8_t* paths, int32_t* plen, int32_t* vl, int32_t* vlen) {
    sel_out o = {leaf, paths, plen, vl, vlen};
    int64_t T = (int64_t)W * C * B;
    for (int64_t s = 0; s < T; s++) {
        int64_t g = s % B;
        int cand = (int)((s / B) % C);
        if (!active[g]) { blank(&o, s); continue; }
        int slot = slots[g * C + cand];
        if (slot < 0 || slot >= max_root) { blank(&o, s); continue; }
        int64_t ri = at(t, g, roots[g]);
        int f = t->fc[ri], n = t->nc[ri];
        if (f < 0 || t->it[ri] || n <= 0 || slot >= n) { blank(&o, s); continue; }
        int node = f + slot;
        if (node < 0 || node >= t->M) { blank(&o, s); continue; }
        int pl = 0, vn = 0;
        if (!det) take_child(t, &o, s, g, node, 0, 0.0f, &pl, &vn);
        else record_move(t, &o, s, at(t, g, node), &pl);
        node = descend(t, &o, s, g, node, 1, c_puct, det, sigma, qp, &pl, &vn);
        leaf[s] = node; plen[s] = pl; vlen[s] = vn;
    }
}

/* mcts_select_with_root_mask_kernel mcts_tree.cuh:689-800 */
void or_mcts_select_mask(const or_tree* t, const int8_t* active, const int32_t* roots, const int8_t* alive,
                         int max_root, float c_puct, int64_t B, int W, int det, float sigma, float qp,
                         int32_t* leaf, uint8_t* paths, int32_t* plen, int32_t* vl, int32_t* vlen) {
    sel_out o = {leaf, paths, plen, vl, vlen};
    int64_t T = (int64_t)W * B;
    for (int64_t s = 0; s < T; s++) {
        int64_t g = s % B;
        if (!active[g]) { blank(&o, s); continue; }
        int node = roots[g], pl = 0, vn = 0;
        int64_t ri = at(t, g, node);
        int f = t->fc[ri], n = t->nc[ri];
        if (!(f < 0 || t->it[ri] || n == 0 || n <= 0 || n > 1024)) {
            int best = puct_argmax(t, g, node, f, n, c_puct, alive + g * max_root, max_root);
            if (best >= 0) {
                node = best;
                take_child(t, &o, s, g, node, 0, 0.0f, &pl, &vn);
                node = descend(t, &o, s, g, node, 1, c_puct, det, sigma, qp, &pl, &vn);
            }
        }
        leaf[s] = node; plen[s] = pl; vlen[s] = vn;
    }
}

/* mcts_replay_kernel mcts_tree.cuh:298-320 */
void or_mcts_replay(const uint8_t* roots, int64_t B, uint8_t* leaves, const uint8_t* paths, const int32_t* plen,
                    const int32_t* leaf, int64_t total) {
    for (int64_t s = 0; s < total; s++) {
        if (leaf[s] < 0) continue;
        uint8_t* row = leaves + s * OR_STATE_BYTES;
        memcpy(row, roots + (s % B) * OR_STATE_BYTES, OR_STATE_BYTES);
        for (int d = 0; d < plen[s] && d < DEPTH; d++) or_apply_move(row, paths + (s * DEPTH + d) * 6);
    }
}

static float result_value(int result, int turn) { /* result_to_value mcts_tree.cuh:182-188 */
    if (result == 3) return 0.0f;
    int p = turn & 1;
    if (result == 1) return p == 0 ? 1.0f : -1.0f;
    if (result == 2) return p == 0 ? -1.0f : 1.0f;
    return 0.0f;
}

/* one simulation's expansion (mcts_expand_dense_priors_kernel :971-1062 body) */
static int expand_one(const or_tree* t, int64_t g, int64_t s, int leaf, const uint8_t* state, const uint8_t* legal,
                      int n, const float* pri, const float* cq, int result) {
    int64_t li = at(t, g, leaf);
    if (result != 0) {
        t->it[li] = 1;
        t->tval[li] = result_value(result, state[3412] | (state[3413] << 8));
        return 0;
    }
    if (t->fc[li] != -1 || n <= 0) return 0;
    int base = t->cnt[g];
    if ((int64_t)base + n > t->M) return 0;
    int ccq, ccr;
    or_centroid(state, &ccq, &ccr);
    for (int m = 0; m < n; m++) {
        int64_t ci = at(t, g, base + m);
        t->vc[ci] = 0;
        t->tv[ci] = 0.0f;
        t->pr[ci] = pri[m];
        t->pa[ci] = leaf;
        t->ai[ci] = or_move_to_action(legal + 6 * m, ccq, ccr);
        t->fc[ci] = -1;
        t->nc[ci] = 0;
        t->it[ci] = 0;
        t->tval[ci] = 0.0f;
        t->ciq[ci] = cq[m];
        memcpy(t->mb + ci * 6, legal + 6 * m, 6);
    }
    t->cnt[g] = base + n;
    t->nc[li] = n;
    t->fc[li] = base;
    (void)s;
    return 1;
}

void or_mcts_expand_dense(const or_tree* t, const float* child_q, const int32_t* leaf, const uint8_t* states,
                          const uint8_t* legal, const int32_t* nlegal, const float* priors, const int32_t* results,
                          int64_t B, int64_t total, int8_t* was) {
    for (int64_t s = 0; s < total; s++) {
        was[s] = 0;
        if (leaf[s] < 0) continue;
        was[s] = (int8_t)expand_one(t, s % B, s, leaf[s], states + s * OR_STATE_BYTES,
                                    legal + s * OR_MAX_LEGAL * 6, nlegal[s], priors + s * OR_MAX_LEGAL,
                                    child_q + s * OR_MAX_LEGAL, results[s]);
    }
}

/* mcts_expand_and_backprop_dense_priors_kernel mcts_tree.cuh:1068-1187 */
void or_mcts_expand_backprop_dense(const or_tree* t, const float* child_q, const int32_t* leaf, const uint8_t* states,
                                   const uint8_t* legal, const int32_t* nlegal, const float* priors,
                                   const int32_t* results, const float* values, const int32_t* vl,
                                   const int32_t* vlen, float qp, int64_t B, int64_t total) {
    for (int64_t s = 0; s < total; s++) {
        if (leaf[s] < 0) continue;
        int64_t g = s % B;
        int e = expand_one(t, g, s, leaf[s], states + s * OR_STATE_BYTES, legal + s * OR_MAX_LEGAL * 6, nlegal[s],
                           priors + s * OR_MAX_LEGAL, child_q + s * OR_MAX_LEGAL, results[s]);
        int64_t li = at(t, g, leaf[s]);
        float v = t->it[li] ? t->tval[li] : (e ? values[s] : 0.0f);
        for (int k = 0; k < vlen[s] && k < DEPTH; k++) {
            int64_t ni = at(t, g, vl[s * DEPTH + k]);
            if (qp > 0.0f) t->vq[ni] += -qp;
            else { t->vc[ni] -= 1; t->tv[ni] += 1.0f; }
        }
        int node = leaf[s];
        for (int k = 0; k < DEPTH + 1 && node >= 0; k++) {
            int64_t ni = at(t, g, node);
            t->vc[ni] += 1;
            t->tv[ni] += v;
            v = -v;
            node = t->pa[ni];
        }
    }
}

/* mcts_root_noise_kernel mcts_tree.cuh:1192-1234 */
void or_mcts_root_noise(const or_tree* t, const float* noise, const int32_t* roots, int pad, float eps, float temp,
                        int64_t B) {
    for (int64_t g = 0; g < B; g++) {
        int64_t ri = at(t, g, roots[g]);
        int f = t->fc[ri], n = t->nc[ri];
        if (f < 0 || n == 0) continue;
        if (temp > 1.0f) {
            float inv = 1.0f / temp, sum = 0.0f;
            for (int c = 0; c < n; c++) {
                float p = powf(t->pr[at(t, g, f + c)], inv);
                t->pr[at(t, g, f + c)] = p;
                sum += p;
            }
            if (sum > 0.0f)
                for (int c = 0; c < n; c++) t->pr[at(t, g, f + c)] /= sum;
        }
        if (eps > 0.0f)
            for (int c = 0; c < n && c < pad; c++) {
                float a = (1.0f - eps) * t->pr[at(t, g, f + c)];
                float b = eps * noise[g * pad + c];
                t->pr[at(t, g, f + c)] = a + b;
            }
    }
}

/* ---- legacy action-space engine (hive_gpu/gpu_native_mcts.py's kernels) ---- */

/* mcts_select_kernel mcts_tree.cuh:205-296: PUCT from the root at every level;
 * the first child stands when no score beats -1e30 */
void or_mcts_select_legacy(const or_tree* t, const int8_t* active, const int32_t* roots, float c_puct, int64_t B,
                           int W, int32_t* leaf, uint8_t* paths, int32_t* plen, int32_t* vl, int32_t* vlen) {
    sel_out o = {leaf, paths, plen, vl, vlen};
    int64_t T = (int64_t)W * B;
    for (int64_t s = 0; s < T; s++) {
        int64_t g = s % B;
        if (!active[g]) { blank(&o, s); continue; }
        int node = roots[g], pl = 0, vn = 0;
        for (int it = 0; it < DEPTH; it++) {
            int64_t ni = at(t, g, node);
            int f = t->fc[ni], n = t->nc[ni];
            if (f < 0 || t->it[ni] || n == 0 || n <= 0 || n > 1024) break;
            int best = f;
            float bs = -1e30f;
            for (int c = 0; c < n; c++) {
                int child = f + c;
                if (child < 0 || child >= t->M) break;
                float sc = puct(t, ni, at(t, g, child), c_puct);
                if (sc > bs) { bs = sc; best = child; }
            }
            node = best;
            take_child(t, &o, s, g, node, 0, 0.0f, &pl, &vn);
        }
        leaf[s] = node; plen[s] = pl; vlen[s] = vn;
    }
}

/* mcts_expand_kernel mcts_tree.cuh:330-433 body: priors from the [ACTION_SPACE]
 * row by action index; moves outside the 17x17 window get no child */
static int expand_legacy_one(const or_tree* t, int64_t g, int leaf, const uint8_t* state, const uint8_t* legal, int n,
                             const float* probs, int result) {
    int64_t li = at(t, g, leaf);
    if (result != 0) {
        t->it[li] = 1;
        t->tval[li] = result_value(result, state[3412] | (state[3413] << 8));
        return 0;
    }
    if (t->fc[li] != -1 || n <= 0) return 0;
    if (n > OR_MAX_LEGAL) n = OR_MAX_LEGAL;
    int base = t->cnt[g];
    if ((int64_t)base + n > t->M) return 0;
    int ccq, ccr;
    or_centroid(state, &ccq, &ccr);
    int created = 0;
    for (int m = 0; m < n; m++) {
        int a = or_move_to_action(legal + 6 * m, ccq, ccr);
        if (a < 0) continue;
        int64_t ci = at(t, g, base + created);
        t->vc[ci] = 0;
        t->tv[ci] = 0.0f;
        t->pr[ci] = probs[a];
        t->pa[ci] = leaf;
        t->ai[ci] = a;
        t->fc[ci] = -1;
        t->nc[ci] = 0;
        t->it[ci] = 0;
        t->tval[ci] = 0.0f;
        memcpy(t->mb + ci * 6, legal + 6 * m, 6);
        created++;
    }
    t->cnt[g] = base + created;
    t->nc[li] = created;
    t->fc[li] = base;
    return 1;
}

enum { ACTIONS = 85834 };

void or_mcts_expand_legacy(const or_tree* t, const int32_t* leaf, const uint8_t* states, const uint8_t* legal,
                           const int32_t* nlegal, const float* probs, const int32_t* results, int64_t B, int64_t total,
                           int8_t* was) {
    for (int64_t s = 0; s < total; s++) {
        was[s] = 0;
        if (leaf[s] < 0) continue;
        was[s] = (int8_t)expand_legacy_one(t, s % B, leaf[s], states + s * OR_STATE_BYTES,
                                           legal + s * OR_MAX_LEGAL * 6, nlegal[s], probs + s * (int64_t)ACTIONS,
                                           results[s]);
    }
}

/* backprop body shared by mcts_backprop_kernel :555-605 and the fused kernel :435-553 */
static void backup_one(const or_tree* t, int64_t g, int64_t s, int leaf, float value_if_expanded, int expanded,
                       const int32_t* vl, const int32_t* vlen) {
    int64_t li = at(t, g, leaf);
    float v = t->it[li] ? t->tval[li] : (expanded ? value_if_expanded : 0.0f);
    for (int k = 0; k < vlen[s] && k < DEPTH; k++) {
        int64_t ni = at(t, g, vl[s * DEPTH + k]);
        t->vc[ni] -= 1;
        t->tv[ni] += 1.0f;
    }
    int node = leaf;
    for (int k = 0; k < DEPTH + 1 && node >= 0; k++) {
        int64_t ni = at(t, g, node);
        t->vc[ni] += 1;
        t->tv[ni] += v;
        v = -v;
        node = t->pa[ni];
    }
}

void or_mcts_backprop_legacy(const or_tree* t, const int32_t* leaf, const float* values, const int32_t* vl,
                             const int32_t* vlen, const int8_t* was, int64_t B, int64_t total) {
    for (int64_t s = 0; s < total; s++)
        if (leaf[s] >= 0) backup_one(t, s % B, s, leaf[s], values[s], was[s] != 0, vl, vlen);
}

void or_mcts_expand_backprop_legacy(const or_tree* t, const int32_t* leaf, const uint8_t* states,
                                    const uint8_t* legal, const int32_t* nlegal, const float* probs,
                                    const int32_t* results, const float* values, const int32_t* vl,
                                    const int32_t* vlen, int64_t B, int64_t total) {
    for (int64_t s = 0; s < total; s++) {
        if (leaf[s] < 0) continue;
        int64_t g = s % B;
        int e = expand_legacy_one(t, g, leaf[s], states + s * OR_STATE_BYTES, legal + s * OR_MAX_LEGAL * 6,
                                  nlegal[s], probs + s * (int64_t)ACTIONS, results[s]);
        backup_one(t, g, s, leaf[s], values[s], e, vl, vlen);
    }
}

/* mcts_extract_policy_kernel mcts_tree.cuh:607-687: policies [B, ACTIONS] zero-filled by the caller */
void or_mcts_extract_policy(const or_tree* t, const int32_t* move_numbers, const int32_t* roots, float temperature,
                            int temp_drop, float pruning, int64_t B, float* policies) {
    for (int64_t g = 0; g < B; g++) {
        float* pol = policies + g * (int64_t)ACTIONS;
        int64_t ri = at(t, g, roots[g]);
        int f = t->fc[ri], n = t->nc[ri];
        if (f < 0 || n == 0) continue;
        float temp = move_numbers[g] >= temp_drop ? 0.0f : temperature;
        if (temp <= 0.0f) {
            int best_a = -1, best_v = -1;
            for (int c = 0; c < n; c++) {
                int64_t ci = at(t, g, f + c);
                if (t->vc[ci] > best_v) { best_v = t->vc[ci]; best_a = t->ai[ci]; }
            }
            if (best_a >= 0 && best_a < ACTIONS) pol[best_a] = 1.0f;
            continue;
        }
        float max_v = 0.0f, sum = 0.0f;
        for (int c = 0; c < n; c++) {
            float v = (float)t->vc[at(t, g, f + c)];
            if (v > max_v) max_v = v;
        }
        for (int c = 0; c < n; c++) {
            int64_t ci = at(t, g, f + c);
            float v = (float)t->vc[ci];
            if (pruning > 0.0f && max_v > 0.0f && v < max_v * pruning) v = 0.0f;
            if (temp != 1.0f) v = powf(v, 1.0f / temp);
            int a = t->ai[ci];
            if (a >= 0 && a < ACTIONS) { pol[a] = v; sum += v; }
        }
        if (sum > 0.0f) {
            for (int c = 0; c < n; c++) {
                int a = t->ai[at(t, g, f + c)];
                if (a >= 0 && a < ACTIONS) pol[a] /= sum;
            }
        } else {
            float u = 1.0f / (float)n;
            for (int c = 0; c < n; c++) {
                int a = t->ai[at(t, g, f + c)];
                if (a >= 0 && a < ACTIONS) pol[a] = u;
            }
        }
    }
}
