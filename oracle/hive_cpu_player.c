/*
 * hive_cpu_player.c -- the reference's CPU search player restated in C: the
 * CPU baseline of the Gumbel self-play configuration.
 *
 * TEST INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg; nothing in
 * hive_neuralnet_amd/ links or calls it).
 *
 * Semantics of FNNNativeCPUPlayer (hive_fnn/fnn_native_cpu_player.py):
 *   _evaluate_state (:126-157): the full legal list and the 122 features of
 *     the node (legal_moves_and_fnn_features), then for every legal move the
 *     child state, its result and its features from the child's FULL legal
 *     list (cpu_native.cpp:130-174, successor_features); the network in fp32
 *     (fnn_network.py: encode = fc2(LayerNorm(sigmoid(fc1 x))), value =
 *     tanh(value_fc e), logit = action_fc2(sigmoid(action_fc1 [e_root | e_child]))),
 *     priors = softmax over the moves;
 *   _expand (:159-181): a finished node returns its result value and stays
 *     unexpanded; otherwise the node is evaluated, gets one child per legal
 *     move and returns the network's value;
 *   _select_child (:183-195): q = -mean(child) (0 unvisited) + c_puct * prior *
 *     sqrt(max(1, N)) / (1 + N(child)), first maximum;
 *   _backpropagate (:197-204): N += 1, W += v, v = -v up to the root;
 *   _run_search_on_existing_root (:206-212) and _gumbel_search (:214-266):
 *     k = min(16, n) candidates by log prior (Gumbel scale 0 by default),
 *     ceil(log2 k) rounds of num_simulations / rounds simulations split over the
 *     candidates (each simulation descends from the candidate child), the top
 *     half kept by log prior + (c_visit + max visits) * c_scale * q, the final
 *     argmax of that score.
 * Tree statistics are doubles, as the reference's Python floats.
 *
 * One difference in storage only: the reference keeps every child's state
 * bytes (3,424 B per legal move of every expanded node); here a child's state
 * is re-derived from its parent's by apply_move when the child is expanded
 * (the same bytes), so a 4,096-simulation search fits in ~15 MB per game.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "hive_oracle.h"

#define CP_H 64  /* hidden / embedding / action width of the `large` preset */

typedef struct {
    int32_t parent, first, count, visits, result, state;  /* state: index into the state arena, -1 = none */
    double total, prior;
    uint8_t move[OR_MOVE_BYTES];
    uint8_t expanded;
} cp_node;

typedef struct {
    cp_node* nodes;
    int64_t n_nodes, cap_nodes;
    uint8_t* states;
    int64_t n_states, cap_states;
    /* scratch of one evaluation */
    uint8_t moves[OR_MAX_LEGAL * OR_MOVE_BYTES];
    uint8_t child_moves[OR_MAX_LEGAL * OR_MOVE_BYTES];
    float root_feat[OR_FEAT_DIM];
    float feat[OR_FEAT_DIM];
    float priors[OR_MAX_LEGAL];
    int32_t results[OR_MAX_LEGAL];
} cp_game;

static float sigmoidf(float x) { return 1.0f / (1.0f + expf(-x)); }

/* encode (fnn_network.py:175-187) of one 122-dim row into e[CP_H] */
static void cp_encode(const or_fnn_weights* w, const float* x, float* e) {
    float h[CP_H];
    for (int o = 0; o < CP_H; o++) {
        const float* row = w->fc1_w + o * OR_FEAT_DIM;
        float s = w->fc1_b[o];
        for (int i = 0; i < OR_FEAT_DIM; i++) s += row[i] * x[i];
        h[o] = sigmoidf(s);
    }
    float mu = 0.0f;
    for (int i = 0; i < CP_H; i++) mu += h[i];
    mu /= (float)CP_H;
    float var = 0.0f;
    for (int i = 0; i < CP_H; i++) var += (h[i] - mu) * (h[i] - mu);
    var /= (float)CP_H;
    const float inv = 1.0f / sqrtf(var + 1e-5f);
    for (int i = 0; i < CP_H; i++) h[i] = (h[i] - mu) * inv * w->ln_w[i] + w->ln_b[i];
    for (int o = 0; o < CP_H; o++) {
        const float* row = w->fc2_w + o * CP_H;
        float s = w->fc2_b[o];
        for (int i = 0; i < CP_H; i++) s += row[i] * h[i];
        e[o] = s;
    }
}

static int32_t cp_new_node(cp_game* G) {
    if (G->n_nodes == G->cap_nodes) {
        G->cap_nodes = G->cap_nodes ? 2 * G->cap_nodes : 4096;
        G->nodes = (cp_node*)realloc(G->nodes, (size_t)G->cap_nodes * sizeof(cp_node));
    }
    cp_node* x = &G->nodes[G->n_nodes];
    memset(x, 0, sizeof(*x));
    x->parent = -1;
    x->first = -1;
    x->state = -1;
    return (int32_t)G->n_nodes++;
}

static int32_t cp_new_state(cp_game* G) {
    if (G->n_states == G->cap_states) {
        G->cap_states = G->cap_states ? 2 * G->cap_states : 1024;
        G->states = (uint8_t*)realloc(G->states, (size_t)G->cap_states * OR_STATE_BYTES);
    }
    return (int32_t)G->n_states++;
}

static uint8_t* cp_state(cp_game* G, int32_t node) {
    cp_node* x = &G->nodes[node];
    if (x->state < 0) {  /* re-derive from the parent's state (the bytes the reference stored) */
        const int32_t s = cp_new_state(G);
        x = &G->nodes[node];
        uint8_t* dst = G->states + (size_t)s * OR_STATE_BYTES;
        memcpy(dst, G->states + (size_t)G->nodes[x->parent].state * OR_STATE_BYTES, OR_STATE_BYTES);
        or_apply_move(dst, x->move);
        x->state = s;
    }
    return G->states + (size_t)x->state * OR_STATE_BYTES;
}

static double cp_result_value(int result, int turn) { /* _result_to_value :117-123 */
    if (result == 0 || result == 3) return 0.0;
    const int white = turn % 2 == 0;
    return ((result == 1 && white) || (result == 2 && !white)) ? 1.0 : -1.0;
}

/* _evaluate_state + the child creation of _expand / _gumbel_search: returns the
 * node's value; the node gets one child per legal move (none when finished). */
static double cp_expand_eval(cp_game* G, const or_fnn_weights* w, int32_t node) {
    uint8_t st[OR_STATE_BYTES];
    memcpy(st, cp_state(G, node), OR_STATE_BYTES);
    const int n = or_legal_moves(st, G->moves);
    or_fnn_features(st, G->moves, n, G->root_feat);
    G->nodes[node].expanded = 1;
    if (n <= 0) return 0.0;
    float er[CP_H], es[CP_H], root_half[CP_H];
    cp_encode(w, G->root_feat, er);
    float v = w->value_b;
    for (int i = 0; i < CP_H; i++) v += w->value_w[i] * er[i];
    const double value = (double)tanhf(v);
    for (int o = 0; o < CP_H; o++) {  /* action_fc1's root half, the same for every move */
        const float* row = w->a1_w + o * 2 * CP_H;
        float s = w->a1_b[o];
        for (int i = 0; i < CP_H; i++) s += row[i] * er[i];
        root_half[o] = s;
    }
    float mx = -INFINITY;
    for (int m = 0; m < n; m++) {
        uint8_t child[OR_STATE_BYTES];
        memcpy(child, st, OR_STATE_BYTES);
        or_apply_move(child, G->moves + m * OR_MOVE_BYTES);
        G->results[m] = child[3415];
        const int cn = or_legal_moves(child, G->child_moves);
        or_fnn_features(child, G->child_moves, cn, G->feat);
        cp_encode(w, G->feat, es);
        float logit = w->a2_b;
        for (int o = 0; o < CP_H; o++) {
            const float* row = w->a1_w + o * 2 * CP_H + CP_H;
            float s = root_half[o];
            for (int i = 0; i < CP_H; i++) s += row[i] * es[i];
            logit += w->a2_w[o] * sigmoidf(s);
        }
        G->priors[m] = logit;
        if (logit > mx) mx = logit;
    }
    float sum = 0.0f;
    for (int m = 0; m < n; m++) sum += (G->priors[m] = expf(G->priors[m] - mx));
    const int32_t first = (int32_t)G->n_nodes;
    for (int m = 0; m < n; m++) {
        const int32_t c = cp_new_node(G);
        cp_node* x = &G->nodes[c];
        x->parent = node;
        x->prior = (double)(G->priors[m] / sum);
        x->result = G->results[m];
        memcpy(x->move, G->moves + m * OR_MOVE_BYTES, OR_MOVE_BYTES);
    }
    G->nodes[node].first = first;
    G->nodes[node].count = n;
    return value;
}

static double cp_mean(const cp_node* x) { return x->visits ? x->total / x->visits : 0.0; }

static void cp_simulate(cp_game* G, const or_fnn_weights* w, int32_t start, double c_puct) {
    int32_t node = start;
    while (G->nodes[node].expanded && G->nodes[node].count > 0) {  /* _select_child */
        const cp_node* p = &G->nodes[node];
        const double sq = sqrt((double)(p->visits > 1 ? p->visits : 1));
        int32_t best = p->first;
        double bs = -1e30;
        for (int32_t c = p->first; c < p->first + p->count; c++) {
            const cp_node* x = &G->nodes[c];
            const double q = x->visits > 0 ? -cp_mean(x) : 0.0;
            const double s = q + c_puct * x->prior * sq / (1 + x->visits);
            if (s > bs) { bs = s; best = c; }
        }
        node = best;
    }
    double v;
    cp_node* x = &G->nodes[node];
    if (x->expanded) v = cp_mean(x);
    else if (x->result != 0) {
        const uint8_t* st = cp_state(G, node);
        v = cp_result_value(G->nodes[node].result, st[3412] | (st[3413] << 8));
    } else v = cp_expand_eval(G, w, node);
    for (int32_t cur = node; cur >= 0; cur = G->nodes[cur].parent) {  /* _backpropagate */
        G->nodes[cur].visits += 1;
        G->nodes[cur].total += v;
        v = -v;
    }
}

/* stable ascending order of score (ties keep index order) */
static void cp_argsort(const double* score, int n, int* idx) {
    for (int i = 0; i < n; i++) idx[i] = i;
    for (int i = 1; i < n; i++) {
        const int k = idx[i];
        int j = i - 1;
        while (j >= 0 && score[idx[j]] > score[k]) { idx[j + 1] = idx[j]; j--; }
        idx[j + 1] = k;
    }
}

/* _gumbel_search (:214-266): returns the chosen slot, -1 without moves; *sims = simulations run */
static int cp_gumbel_search(cp_game* G, const or_fnn_weights* w, const uint8_t* root_state, int num_sims,
                            int considered, double c_puct, double c_visit, double c_scale, int64_t* sims) {
    G->n_nodes = 0;
    G->n_states = 0;
    const int32_t root = cp_new_node(G);
    const int32_t s = cp_new_state(G);
    memcpy(G->states + (size_t)s * OR_STATE_BYTES, root_state, OR_STATE_BYTES);
    G->nodes[root].state = s;
    cp_expand_eval(G, w, root);
    const int n = G->nodes[root].count;
    if (n <= 0) return -1;
    const int32_t first = G->nodes[root].first;
    const int k = considered < n ? considered : n;
    int rounds = 1;
    while ((1 << rounds) < k) rounds++;  /* max(1, ceil(log2 k)) */
    const int per_round = num_sims / rounds > 1 ? num_sims / rounds : 1;
    double base[OR_MAX_LEGAL];
    for (int m = 0; m < n; m++) {
        const double p = G->nodes[first + m].prior;
        base[m] = log(p > 1e-30 ? p : 1e-30);
    }
    int order[OR_MAX_LEGAL], cand[OR_MAX_LEGAL] = {0}, nc = k;
    cp_argsort(base, n, order);  /* argsort(base)[-k:][::-1] */
    for (int i = 0; i < k; i++) cand[i] = order[n - 1 - i];
    for (int r = 0; r < rounds && nc > 1; r++) {
        const int spc = per_round / nc > 1 ? per_round / nc : 1;
        double cs[OR_MAX_LEGAL];
        double vmax = 0.0;
        for (int i = 0; i < nc; i++) {
            const int32_t c = first + cand[i];
            for (int t = 0; t < spc; t++) cp_simulate(G, w, c, c_puct);
            *sims += spc;
            if (G->nodes[c].visits > vmax) vmax = G->nodes[c].visits;
        }
        const double sigma = (c_visit + vmax) * c_scale;
        for (int i = 0; i < nc; i++) cs[i] = (float)(base[cand[i]] + sigma * (float)(-cp_mean(&G->nodes[first + cand[i]])));
        const int keep = nc / 2 > 1 ? nc / 2 : 1;
        int o2[OR_MAX_LEGAL], nxt[OR_MAX_LEGAL];
        cp_argsort(cs, nc, o2);
        for (int i = 0; i < keep; i++) nxt[i] = cand[o2[nc - 1 - i]];
        for (int i = 0; i < keep; i++) cand[i] = nxt[i];
        nc = keep;
    }
    if (nc == 1) return cand[0];
    double vmax = 0.0;
    for (int i = 0; i < nc; i++)
        if (G->nodes[first + cand[i]].visits > vmax) vmax = G->nodes[first + cand[i]].visits;
    const double sigma = (c_visit + vmax) * c_scale;
    int best = cand[0];
    double bs = -1e300;
    for (int i = 0; i < nc; i++) {
        const double sc = (float)(base[cand[i]] + sigma * (float)(-cp_mean(&G->nodes[first + cand[i]])));
        if (sc > bs) { bs = sc; best = cand[i]; }
    }
    return best;
}

typedef struct {
    const uint8_t* states;
    const or_fnn_weights* w;
    int num_sims, considered;
    double c_puct, c_visit, c_scale;
    int32_t* chosen;
    int64_t* sims;
    int64_t lo, hi;
} cp_span;

static void* cp_run(void* p) {
    cp_span* sp = (cp_span*)p;
    cp_game G;
    memset(&G, 0, sizeof(G));
    for (int64_t g = sp->lo; g < sp->hi; g++) {
        int64_t s = 0;
        sp->chosen[g] = cp_gumbel_search(&G, sp->w, sp->states + g * OR_STATE_BYTES, sp->num_sims, sp->considered,
                                         sp->c_puct, sp->c_visit, sp->c_scale, &s);
        sp->sims[g] = s;
    }
    free(G.nodes);
    free(G.states);
    return NULL;
}

void or_cpu_player_search(const uint8_t* states, int64_t G, const or_fnn_weights* w, int num_sims, int considered,
                          float c_puct, float c_visit, float c_scale, int32_t* chosen, int64_t* sims, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    if (threads > G) threads = (int)(G > 0 ? G : 1);
    pthread_t tid[256];
    cp_span sp[256];
    for (int t = 0; t < threads; t++) {
        sp[t] = (cp_span){states, w, num_sims, considered, c_puct, c_visit, c_scale, chosen, sims,
                          G * t / threads, G * (t + 1) / threads};
        pthread_create(&tid[t], NULL, cp_run, &sp[t]);
    }
    for (int t = 0; t < threads; t++) pthread_join(tid[t], NULL);
}
