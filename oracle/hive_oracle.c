/*
 * hive_oracle.c -- CPU restatement of the reference's batched Hive engine.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the parity checker for the HIP product
 * path (hive_neuralnet_amd/csrc).  It is loaded only by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg.  The product
 * never calls it and must fail loudly when its HIP library is missing.
 *
 * Every function restates one reference function; the citation names the
 * file:line under chrismejias/hive_neuralnet it follows.  The restatement is
 * pinned three ways (see tests/test_oracle_*.py):
 *   - golden vectors written by the reference's own C++ headers compiled in
 *     this container (oracle/ref_capi.cpp, tests/golden/),
 *   - known-answer rule cases restated from the reference's Python tests,
 *   - closed forms / brute force (hex tables, articulation points by vertex
 *     deletion, banker's rounding, action-index formula).
 *
 * Parity status per function is recorded in tests/test_oracle_pins.py.
 */
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "hive_oracle.h"

enum {
    NCELL = 529, GRID = 23, HALF = 11, NDIR = 6, NWORD = 9,
    MAXLEG = 256, MAXSTACK = 5, ANTCAP = 128, SMALLCAP = 32,
    CENTER_CELL = HALF * GRID + HALF,
};

enum { PT_NONE = 0, PT_Q = 1, PT_A = 2, PT_G = 3, PT_S = 4, PT_B = 5, PT_M = 6, PT_L = 7, PT_P = 8 };
enum { MV_PLACE = 0, MV_MOVE = 1, MV_PASS = 2 };
enum { RES_NONE = 0, RES_WHITE = 1, RES_BLACK = 2, RES_DRAW = 3 };

/* ---- byte layout (hive_gpu/csrc/hive_state.cuh:239-269; offsets probe-verified) ---- */
typedef struct {
    uint8_t stack[MAXSTACK][NCELL]; /* @0    level-major piece bytes: type | color<<4 */
    uint8_t height[NCELL];          /* @2645 */
    uint8_t pad0[2];                /* @3174 */
    uint64_t occ[NWORD];            /* @3176 */
    uint64_t wtop[NWORD];           /* @3248 */
    uint64_t btop[NWORD];           /* @3320 */
    uint16_t queen[2];              /* @3392 0xFFFF = not placed */
    uint8_t hand[2][8];             /* @3396 index = type-1 */
    uint16_t turn;                  /* @3412 */
    uint8_t qplaced;                /* @3414 bit c = colour c's queen placed */
    uint8_t result;                 /* @3415 */
    uint16_t stun;                  /* @3416 0xFFFF = none */
    int8_t cq, cr;                  /* @3418 always 0 */
    uint8_t pad1[4];                /* @3420 */
} hstate;

typedef struct {
    uint8_t type, pt;
    uint16_t from, to;
} hmove;

_Static_assert(sizeof(hstate) == OR_STATE_BYTES, "state size");
_Static_assert(__builtin_offsetof(hstate, height) == 2645, "height");
_Static_assert(__builtin_offsetof(hstate, occ) == 3176, "occ");
_Static_assert(__builtin_offsetof(hstate, wtop) == 3248, "wtop");
_Static_assert(__builtin_offsetof(hstate, btop) == 3320, "btop");
_Static_assert(__builtin_offsetof(hstate, queen) == 3392, "queen");
_Static_assert(__builtin_offsetof(hstate, hand) == 3396, "hand");
_Static_assert(__builtin_offsetof(hstate, turn) == 3412, "turn");
_Static_assert(__builtin_offsetof(hstate, qplaced) == 3414, "qplaced");
_Static_assert(__builtin_offsetof(hstate, result) == 3415, "result");
_Static_assert(__builtin_offsetof(hstate, stun) == 3416, "stun");
_Static_assert(sizeof(hmove) == OR_MOVE_BYTES, "move size");

static const uint8_t PER_TYPE[8] = {1, 3, 3, 2, 2, 1, 1, 1}; /* hive_state.cuh:52-61 */

/* ---- geometry: closed form of hive_gpu/csrc/hex_grid.cuh:41-49,69-108 ---- */
static int16_t NB[NCELL][NDIR];
static const int DCOL[NDIR] = {+1, +1, 0, -1, -1, 0}; /* E NE NW W SW SE */
static const int DROW[NDIR] = {0, -1, -1, 0, +1, +1};

__attribute__((constructor)) static void build_tables(void) {
    for (int c = 0; c < NCELL; c++) {
        int row = c / GRID, col = c % GRID;
        for (int d = 0; d < NDIR; d++) {
            int r2 = row + DROW[d], c2 = col + DCOL[d];
            NB[c][d] = (r2 >= 0 && r2 < GRID && c2 >= 0 && c2 < GRID) ? (int16_t)(r2 * GRID + c2) : -1;
        }
    }
}
/* slide flanks: dest = NB[c][d], cw = NB[c][(d+5)%6], ccw = NB[c][(d+1)%6] */
static inline int cw_of(int c, int d) { return NB[c][(d + 5) % 6]; }
static inline int ccw_of(int c, int d) { return NB[c][(d + 1) % 6]; }

/* ---- bit helpers ---- */
static inline int bget(const uint64_t* w, int c) { return (int)((w[c >> 6] >> (c & 63)) & 1u); }
static inline void bset(uint64_t* w, int c) { w[c >> 6] |= 1ull << (c & 63); }
static inline void bclr(uint64_t* w, int c) { w[c >> 6] &= ~(1ull << (c & 63)); }
static inline int bpop(const uint64_t* w) {
    int n = 0;
    for (int i = 0; i < NWORD; i++) n += __builtin_popcountll(w[i]);
    return n;
}
/* iterate set bits of a 9-word board in ascending cell order */
#define FOR_EACH_BIT(words, cellvar)                                              \
    for (int _wi = 0; _wi < NWORD; _wi++)                                         \
        for (uint64_t _b = (words)[_wi]; _b; _b &= _b - 1)                        \
            for (int cellvar = _wi * 64 + __builtin_ctzll(_b), _once = 1; _once; _once = 0) \
                if (cellvar < NCELL)

static inline int occ_at(const hstate* s, int c) { return bget(s->occ, c); }
static inline uint8_t top_byte(const hstate* s, int c) {
    int h = s->height[c];
    return h ? s->stack[h - 1][c] : 0;
}
static inline int top_type(const hstate* s, int c) { return top_byte(s, c) & 15; }
static inline int top_color(const hstate* s, int c) { return (top_byte(s, c) >> 4) & 1; }
static inline int side_to_move(const hstate* s) { return s->turn & 1; }
static inline int queen_down(const hstate* s, int c) { return (s->qplaced >> c) & 1; }
static inline int is_stunned(const hstate* s, int c) { return s->stun != 0xFFFF && (int)s->stun == c; }

static int occupied_neighbours(const hstate* s, int c) { /* hive_state.cuh:314-321 */
    int n = 0;
    for (int d = 0; d < NDIR; d++) {
        int nb = NB[c][d];
        if (nb >= 0 && occ_at(s, nb)) n++;
    }
    return n;
}

/* ---- state mutation: hive_state.cuh:326-517 ---- */
static void set_top_colour(hstate* s, int c, int colour) {
    if (colour == 0) { bset(s->wtop, c); bclr(s->btop, c); }
    else { bset(s->btop, c); bclr(s->wtop, c); }
}

static void push_piece(hstate* s, int c, int pt, int colour) { /* place_piece :326-359 */
    int h = s->height[c];
    if (h >= MAXSTACK || c < 0 || c >= NCELL) return;
    s->stack[h][c] = (uint8_t)(pt | (colour << 4));
    s->height[c] = (uint8_t)(h + 1);
    if (h == 0) bset(s->occ, c);
    set_top_colour(s, c, colour);
    if (pt == PT_Q) {
        s->queen[colour] = (uint16_t)c;
        s->qplaced |= (uint8_t)(1 << colour);
    }
    s->hand[colour][pt - 1]--;
}

static uint8_t pop_piece(hstate* s, int c) { /* remove_top :365-391 */
    int h = s->height[c];
    if (h <= 0 || c < 0 || c >= NCELL) return 0;
    uint8_t b = s->stack[h - 1][c];
    s->stack[h - 1][c] = 0;
    s->height[c] = (uint8_t)(h - 1);
    if (h == 1) {
        bclr(s->occ, c); bclr(s->wtop, c); bclr(s->btop, c);
    } else {
        set_top_colour(s, c, (s->stack[h - 2][c] >> 4) & 1);
    }
    return b;
}

static void relocate(hstate* s, int from, int to) { /* move_piece :397-428 */
    if (from < 0 || from >= NCELL || to < 0 || to >= NCELL) return;
    if (s->height[from] <= 0) return;
    if (s->height[to] >= MAXSTACK) return;
    uint8_t b = pop_piece(s, from);
    int pt = b & 15, colour = (b >> 4) & 1;
    int h = s->height[to];
    s->stack[h][to] = b;
    s->height[to] = (uint8_t)(h + 1);
    if (h == 0) bset(s->occ, to);
    set_top_colour(s, to, colour);
    if (pt == PT_Q) s->queen[colour] = (uint16_t)to;
}

static int queen_ringed(const hstate* s, int colour) { /* is_queen_surrounded :433-437 */
    if (!queen_down(s, colour)) return 0;
    return occupied_neighbours(s, s->queen[colour]) == 6;
}

static void update_result(hstate* s) { /* check_game_over :442-448 */
    int w = queen_ringed(s, 0), b = queen_ringed(s, 1);
    if (w && b) s->result = RES_DRAW;
    else if (w) s->result = RES_BLACK;
    else if (b) s->result = RES_WHITE;
}

void or_init_state(uint8_t* raw, int mask) { /* init_state :454-492 on a zero-filled row */
    hstate* s = (hstate*)raw;
    memset(s, 0, sizeof(*s));
    s->queen[0] = s->queen[1] = 0xFFFF;
    for (int c = 0; c < 2; c++) {
        for (int p = 0; p < 5; p++) s->hand[c][p] = PER_TYPE[p];
        s->hand[c][5] = (mask & 1) ? 1 : 0;
        s->hand[c][6] = (mask & 2) ? 1 : 0;
        s->hand[c][7] = (mask & 4) ? 1 : 0;
    }
    s->stun = 0xFFFF;
}

static void apply(hstate* s, const hmove* m) { /* apply_move :497-517 */
    if (m->type == MV_PLACE) {
        if (m->to < NCELL && m->pt >= PT_Q && m->pt <= PT_P) push_piece(s, m->to, m->pt, side_to_move(s));
        s->stun = 0xFFFF;
    } else if (m->type == MV_MOVE) {
        if (m->from < NCELL && m->to < NCELL) {
            relocate(s, m->from, m->to);
            s->stun = m->to;
        }
    } else {
        s->stun = 0xFFFF;
    }
    s->turn++;
    update_result(s);
}

void or_apply_move(uint8_t* raw, const uint8_t* mv) {
    hmove m;
    memcpy(&m, mv, sizeof(m));
    apply((hstate*)raw, &m);
}

/* ---- articulation points: articulation.cuh:34-168 ----
 * The reference runs Tarjan's DFS from the lowest occupied cell only, so
 * the result is the articulation-point set of that cell's connected
 * component (other components contribute nothing); <= 2 occupied cells
 * yields the empty set.  Restated as an iterative low-link DFS. */
static void articulation(const hstate* s, uint64_t* ap) {
    memset(ap, 0, NWORD * sizeof(uint64_t));
    int cells[28], n = 0;
    FOR_EACH_BIT(s->occ, c) {
        if (n < 28) cells[n++] = c;
    }
    if (n <= 2) return;
    int8_t index_of[NCELL];
    memset(index_of, -1, sizeof(index_of));
    for (int i = 0; i < n; i++) index_of[cells[i]] = (int8_t)i;
    int order[28], low[28], par[28], kids[28], next_dir[28], stack[28];
    for (int i = 0; i < n; i++) { order[i] = -1; par[i] = -1; kids[i] = 0; }
    int clock = 0, sp = 0;
    order[0] = low[0] = clock++;
    next_dir[0] = 0;
    stack[sp++] = 0;
    while (sp) {
        int u = stack[sp - 1];
        if (next_dir[u] < NDIR) {
            int d = next_dir[u]++;
            int nb = NB[cells[u]][d];
            if (nb < 0 || !occ_at(s, nb) || index_of[nb] < 0) continue;
            int v = index_of[nb];
            if (order[v] < 0) {
                par[v] = u; kids[u]++;
                order[v] = low[v] = clock++;
                next_dir[v] = 0;
                stack[sp++] = v;
            } else if (v != par[u] && order[v] < low[u]) {
                low[u] = order[v];
            }
        } else {
            sp--;
            if (!sp) break;
            int p = stack[sp - 1];
            if (low[u] < low[p]) low[p] = low[u];
            if (par[p] < 0) { if (kids[p] > 1) bset(ap, cells[p]); }
            else if (low[u] >= order[p]) bset(ap, cells[p]);
        }
    }
}

void or_articulation(const uint8_t* raw, uint64_t* ap) { articulation((const hstate*)raw, ap); }

/* per-position cache: init_movegen_state_cache move_gen.cuh:161-178 */
typedef struct {
    uint64_t ap[NWORD];
    uint64_t pinned[NWORD];
    uint64_t perim[NWORD]; /* build_empty_perimeter_mask :133-152 over the full occupancy */
} pos_cache;

static void cache_init(const hstate* s, pos_cache* k) {
    articulation(s, k->ap);
    memset(k->pinned, 0, sizeof(k->pinned));
    FOR_EACH_BIT(k->ap, c) {
        if (s->height[c] == 1) bset(k->pinned, c);
    }
    memset(k->perim, 0, sizeof(k->perim));
    FOR_EACH_BIT(s->occ, c) {
        for (int d = 0; d < NDIR; d++) {
            int nb = NB[c][d];
            if (nb >= 0 && !occ_at(s, nb)) bset(k->perim, nb);
        }
    }
}

/* ---- slide rules ---- */
/* can_slide :82-104 -- `ghost` is treated as empty */
static int slide_ok(const hstate* s, int from, int d, int ghost) {
    int dest = NB[from][d];
    if (dest < 0) return 0;
    if (occ_at(s, dest) && dest != ghost) return 0;
    int a = cw_of(from, d), b = ccw_of(from, d);
    int ao = a >= 0 && occ_at(s, a) && a != ghost;
    int bo = b >= 0 && occ_at(s, b) && b != ghost;
    return ao != bo;
}

/* can_slide_ant_occ :120-131 */
static int ant_step_ok(const uint64_t* occ, const uint64_t* perim, int from, int d) {
    int dest = NB[from][d];
    if (dest < 0 || !bget(perim, dest)) return 0;
    int a = cw_of(from, d), b = ccw_of(from, d);
    int ao = a >= 0 && bget(occ, a);
    int bo = b >= 0 && bget(occ, b);
    return ao != bo;
}

/* elevated_gate_blocked :659-667 */
static int high_gate(const hstate* s, int from, int d, int h) {
    int a = cw_of(from, d), b = ccw_of(from, d);
    int ah = a >= 0 ? s->height[a] : 0;
    int bh = b >= 0 ? s->height[b] : 0;
    return ah > h && bh > h;
}

static int dir_between(int from, int to) { /* find_direction :673-678 */
    for (int d = 0; d < NDIR; d++)
        if (NB[from][d] == to) return d;
    return -1;
}

static inline int imax(int a, int b) { return a > b ? a : b; }

/* ---- per-type destination generators (dest cells in reference order) ---- */
static int dests_step(const hstate* s, int c, uint16_t* out) { /* gen_queen_moves :202-212 */
    int n = 0;
    for (int d = 0; d < NDIR; d++)
        if (slide_ok(s, c, d, c)) out[n++] = (uint16_t)NB[c][d];
    return n;
}

static int dests_hopper(const hstate* s, int c, uint16_t* out) { /* gen_grasshopper_moves :228-245 */
    int n = 0;
    for (int d = 0; d < NDIR; d++) {
        int p = NB[c][d];
        if (p < 0 || !occ_at(s, p)) continue;
        while (p >= 0 && occ_at(s, p)) p = NB[p][d];
        if (p >= 0) out[n++] = (uint16_t)p;
    }
    return n;
}

/* Ant flood fill: FIFO breadth-first search over ground slides with the ant
 * lifted, seeded in direction order, each queue entry expanded in direction
 * order (gen_ant_moves_with_perimeter :267-313 and
 * emit_ant_moves_with_perimeter :348-388 -- both are this search cut off
 * after `cap` discoveries). */
static int dests_ant(const hstate* s, int c, const uint64_t* perim, uint16_t* out, int cap) {
    if (cap <= 0) return 0;
    uint64_t occ[NWORD], seen[NWORD];
    memcpy(occ, s->occ, sizeof(occ));
    bclr(occ, c);
    memset(seen, 0, sizeof(seen));
    bset(seen, c);
    int head = 0, tail = 0;
    for (int d = 0; d < NDIR && tail < cap; d++) {
        if (!ant_step_ok(occ, perim, c, d)) continue;
        int dest = NB[c][d];
        if (bget(seen, dest)) continue;
        bset(seen, dest);
        out[tail++] = (uint16_t)dest;
    }
    while (head < tail && tail < cap) {
        int cur = out[head++];
        for (int d = 0; d < NDIR && tail < cap; d++) {
            if (!ant_step_ok(occ, perim, cur, d)) continue;
            int dest = NB[cur][d];
            if (bget(seen, dest)) continue;
            bset(seen, dest);
            out[tail++] = (uint16_t)dest;
        }
    }
    return tail;
}

static int dests_spider(const hstate* s, int c, uint16_t* out) { /* gen_spider_moves :397-431 */
    uint64_t got[NWORD] = {0};
    int n = 0;
    for (int d1 = 0; d1 < NDIR; d1++) {
        if (!slide_ok(s, c, d1, c)) continue;
        int p1 = NB[c][d1];
        for (int d2 = 0; d2 < NDIR; d2++) {
            if (!slide_ok(s, p1, d2, c)) continue;
            int p2 = NB[p1][d2];
            if (p2 == c || p2 == p1) continue;
            for (int d3 = 0; d3 < NDIR; d3++) {
                if (!slide_ok(s, p2, d3, c)) continue;
                int p3 = NB[p2][d3];
                if (p3 == c || p3 == p1 || p3 == p2) continue;
                if (!bget(got, p3) && n < SMALLCAP) {
                    bset(got, p3);
                    out[n++] = (uint16_t)p3;
                }
            }
        }
    }
    return n;
}

static int dests_beetle(const hstate* s, int c, uint16_t* out) { /* gen_beetle_moves :468-502 */
    int n = 0, below = s->height[c] - 1;
    for (int d = 0; d < NDIR; d++) {
        int dest = NB[c][d];
        if (dest < 0) continue;
        int h = imax(s->height[dest], below);
        if (h > 0) {
            if (!high_gate(s, c, d, h)) out[n++] = (uint16_t)dest;
        } else if (slide_ok(s, c, d, c)) {
            out[n++] = (uint16_t)dest;
        }
    }
    return n;
}

static int dests_ladybug(const hstate* s, int c, uint16_t* out) { /* gen_ladybug_moves :538-596 */
    uint64_t got[NWORD] = {0};
    int n = 0;
    for (int d1 = 0; d1 < NDIR; d1++) {
        int p1 = NB[c][d1];
        if (p1 < 0 || !occ_at(s, p1)) continue;
        if (high_gate(s, c, d1, imax(s->height[c] - 1, s->height[p1]))) continue;
        for (int d2 = 0; d2 < NDIR; d2++) {
            int p2 = NB[p1][d2];
            if (p2 < 0 || p2 == c || !occ_at(s, p2)) continue;
            if (high_gate(s, p1, d2, imax(s->height[p1], s->height[p2]))) continue;
            for (int d3 = 0; d3 < NDIR; d3++) {
                int p3 = NB[p2][d3];
                if (p3 < 0 || p3 == c || p3 == p1 || occ_at(s, p3)) continue;
                if (high_gate(s, p2, d3, imax(s->height[p2], 0))) continue;
                if (!bget(got, p3) && n < SMALLCAP) {
                    bset(got, p3);
                    out[n++] = (uint16_t)p3;
                }
            }
        }
    }
    return n;
}

/* gen_mosquito_moves :907-1008: beetle when elevated, else the deduplicated
 * union of the abilities of adjacent non-mosquito top pieces, in the order
 * Q/P, A, G, S, B, L, capped at 128. */
static int dests_mosquito(const hstate* s, int c, const uint64_t* perim, uint16_t* out) {
    if (s->height[c] > 1) return dests_beetle(s, c, out);
    int has[9] = {0};
    for (int d = 0; d < NDIR; d++) {
        int nb = NB[c][d];
        if (nb < 0 || !occ_at(s, nb)) continue;
        int t = top_type(s, nb);
        if (t != PT_M) has[t] = 1;
    }
    uint64_t got[NWORD] = {0};
    uint16_t tmp[ANTCAP];
    int n = 0;
    for (int k = 0; k < 6; k++) {
        int m = 0;
        switch (k) {
            case 0: if (has[PT_Q] || has[PT_P]) m = dests_step(s, c, tmp); break;
            case 1: if (has[PT_A]) m = dests_ant(s, c, perim, tmp, ANTCAP); break;
            case 2: if (has[PT_G]) m = dests_hopper(s, c, tmp); break;
            case 3: if (has[PT_S]) m = dests_spider(s, c, tmp); break;
            case 4: if (has[PT_B]) m = dests_beetle(s, c, tmp); break;
            case 5: if (has[PT_L]) m = dests_ladybug(s, c, tmp); break;
        }
        for (int i = 0; i < m; i++) {
            if (bget(got, tmp[i])) continue;
            bset(got, tmp[i]);
            if (n < ANTCAP) out[n++] = tmp[i];
        }
    }
    return n;
}

/* One pillbug-ability actor at `pc` throwing target `t` (gen_pillbug_throws
 * :691-740 per-target body).  Writes drop cells in direction order; returns
 * count (0 when the target is not throwable). */
static int throw_drops(const hstate* s, const pos_cache* k, int pc, int t, uint16_t* drops) {
    if (t < 0 || !occ_at(s, t)) return 0;
    if (s->height[t] != 1) return 0;
    if (is_stunned(s, t)) return 0;
    if (bget(k->pinned, t)) return 0;
    int ph = s->height[pc];
    int back = dir_between(t, pc);
    if (back < 0) return 0;
    if (high_gate(s, t, back, imax(s->height[t] - 1, ph))) return 0;
    int n = 0;
    for (int dd = 0; dd < NDIR; dd++) {
        int dest = NB[pc][dd];
        if (dest < 0 || dest == t || occ_at(s, dest)) continue;
        if (high_gate(s, pc, dd, imax(ph, 0))) continue;
        drops[n++] = (uint16_t)dest;
    }
    return n;
}

static int next_to_top_pillbug(const hstate* s, int c) {
    for (int d = 0; d < NDIR; d++) {
        int nb = NB[c][d];
        if (nb >= 0 && occ_at(s, nb) && top_type(s, nb) == PT_P) return 1;
    }
    return 0;
}

/* find_placement_positions :1064-1140 */
static int placement_cells(const hstate* s, int colour, uint64_t* out) {
    memset(out, 0, NWORD * sizeof(uint64_t));
    if (s->turn == 0) { bset(out, CENTER_CELL); return 1; }
    int n = 0;
    if (s->turn == 1) {
        FOR_EACH_BIT(s->occ, c) {
            for (int d = 0; d < NDIR; d++) {
                int nb = NB[c][d];
                if (nb >= 0 && !occ_at(s, nb)) { bset(out, nb); n++; }
            }
        }
        return n;
    }
    const uint64_t* mine = colour ? s->btop : s->wtop;
    const uint64_t* theirs = colour ? s->wtop : s->btop;
    uint64_t tried[NWORD] = {0};
    FOR_EACH_BIT(mine, c) {
        for (int d = 0; d < NDIR; d++) {
            int nb = NB[c][d];
            if (nb < 0 || occ_at(s, nb) || bget(tried, nb)) continue;
            bset(tried, nb);
            int bad = 0;
            for (int d2 = 0; d2 < NDIR && !bad; d2++) {
                int x = NB[nb][d2];
                if (x >= 0 && bget(theirs, x)) bad = 1;
            }
            if (!bad) { bset(out, nb); n++; }
        }
    }
    return n;
}

static inline void put_move(hmove* out, int i, int type, int pt, int from, int to) {
    out[i].type = (uint8_t)type;
    out[i].pt = (uint8_t)pt;
    out[i].from = (uint16_t)from;
    out[i].to = (uint16_t)to;
}

/* generate_legal_moves :1151-1360 */
static int legal_moves(const hstate* s, hmove* out) {
    if (s->result != RES_NONE) return 0;
    int me = side_to_move(s), my_turn = s->turn / 2, n = 0;
    int queen_now = (my_turn == 3 && !queen_down(s, me));
    int placeable[8], any = 0;
    for (int p = 0; p < 8; p++) {
        placeable[p] = queen_now ? (p == 0 && s->hand[me][0] > 0) : (s->hand[me][p] > 0);
        any |= placeable[p];
    }
    if (any) {
        uint64_t cells[NWORD];
        if (placement_cells(s, me, cells) > 0) {
            FOR_EACH_BIT(cells, c) {
                for (int p = 0; p < 8; p++) {
                    if (!placeable[p] || (my_turn == 0 && p == 0)) continue;
                    if (n < MAXLEG) put_move(out, n++, MV_PLACE, p + 1, 0, c);
                }
            }
        }
    }
    if (queen_down(s, me)) {
        pos_cache k;
        cache_init(s, &k);
        const uint64_t* mine = me ? s->btop : s->wtop;
        FOR_EACH_BIT(mine, c) {
            if (is_stunned(s, c) || bget(k.pinned, c)) continue;
            int pt = top_type(s, c);
            if (pt == PT_A) {
                /* ants write straight into the list (cap = what is left of 256) */
                uint16_t tmp[MAXLEG];
                int m = dests_ant(s, c, k.perim, tmp, MAXLEG - n);
                for (int i = 0; i < m; i++) put_move(out, n++, MV_MOVE, PT_A, c, tmp[i]);
                continue;
            }
            uint16_t dst[ANTCAP];
            int m = 0;
            switch (pt) {
                case PT_Q: m = dests_step(s, c, dst); break;
                case PT_G: m = dests_hopper(s, c, dst); break;
                case PT_S: m = dests_spider(s, c, dst); break;
                case PT_B: m = dests_beetle(s, c, dst); break;
                case PT_M: m = dests_mosquito(s, c, k.perim, dst); break;
                case PT_L: m = dests_ladybug(s, c, dst); break;
                case PT_P: m = dests_step(s, c, dst); break;
                default: break;
            }
            for (int i = 0; i < m && n < MAXLEG; i++) put_move(out, n++, MV_MOVE, pt, c, dst[i]);
        }
        /* throws: own top pillbugs (stun and pin not checked on the thrower),
         * then own ground mosquitoes touching any top pillbug (:1304-1345) */
        FOR_EACH_BIT(mine, c) {
            int pt = top_type(s, c);
            int actor = (pt == PT_P) || (pt == PT_M && s->height[c] == 1 && next_to_top_pillbug(s, c));
            if (!actor) continue;
            for (int dt = 0; dt < NDIR; dt++) {
                int t = NB[c][dt];
                uint16_t drops[NDIR];
                int m = throw_drops(s, &k, c, t, drops);
                for (int i = 0; i < m; i++)
                    if (n < MAXLEG) put_move(out, n++, MV_MOVE, top_type(s, t), t, drops[i]);
            }
        }
    }
    if (n == 0) { put_move(out, 0, MV_PASS, 0, 0, 0); n = 1; }
    return n;
}

/* ---- compact successor list: generate_fnn_feature_moves :1416-1563 ---- */
static int piece_can_move(const hstate* s, const pos_cache* k, int c, int pt) {
    uint16_t tmp[MAXLEG];
    switch (pt) { /* the reference's has_*_move predicates == "generator non-empty" */
        case PT_Q: case PT_P: return dests_step(s, c, tmp) > 0;
        case PT_A: return dests_ant(s, c, k->perim, tmp, 1) > 0;
        case PT_G: return dests_hopper(s, c, tmp) > 0;
        case PT_S: return dests_spider(s, c, tmp) > 0;
        case PT_B: return dests_beetle(s, c, tmp) > 0;
        case PT_M: return dests_mosquito(s, c, k->perim, tmp) > 0;
        case PT_L: return dests_ladybug(s, c, tmp) > 0;
        default: return 0;
    }
}

/* emit_fnn_move_flag :1362-1377 */
static void flag_move(const hstate* s, hmove* out, int* n, uint32_t* seen, int pt, int from) {
    int h = s->height[from];
    if (h <= 0) return;
    int owner = (s->stack[h - 1][from] >> 4) & 1;
    int bit = (pt - 1) * 2 + owner;
    if (*seen & (1u << bit)) return;
    *seen |= 1u << bit;
    put_move(out, (*n)++, MV_MOVE, pt, from, 0);
}

static int compact_moves(const hstate* s, hmove* out) {
    if (s->result != RES_NONE) return 0;
    int me = side_to_move(s), my_turn = s->turn / 2, n = 0;
    int queen_now = (my_turn == 3 && !queen_down(s, me));
    int any = 0;
    for (int p = 0; p < 8; p++) {
        int ok = queen_now ? (p == 0 && s->hand[me][0] > 0) : (s->hand[me][p] > 0);
        if (my_turn == 0 && p == 0) ok = 0;
        any |= ok;
    }
    if (any) {
        uint64_t cells[NWORD];
        if (placement_cells(s, me, cells) > 0) {
            FOR_EACH_BIT(cells, c) {
                if (n < MAXLEG) put_move(out, n++, MV_PLACE, 0, 0, c);
            }
        }
    }
    if (!queen_down(s, me) || n >= MAXLEG) {
        if (n == 0) { put_move(out, 0, MV_PASS, 0, 0, 0); return 1; }
        return n;
    }
    pos_cache k;
    cache_init(s, &k);
    uint32_t seen = 0;
    const uint64_t* mine = me ? s->btop : s->wtop;
    FOR_EACH_BIT(mine, c) {
        if (n >= MAXLEG) continue; /* the reference stops scanning once the list is full */
        if (is_stunned(s, c) || bget(k.pinned, c)) continue;
        int pt = top_type(s, c);
        if (seen & (1u << ((pt - 1) * 2 + me))) continue;
        if (piece_can_move(s, &k, c, pt)) flag_move(s, out, &n, &seen, pt, c);
    }
    FOR_EACH_BIT(mine, c) {
        if (n >= MAXLEG) continue;
        int pt = top_type(s, c);
        int actor = (pt == PT_P) || (pt == PT_M && s->height[c] == 1 && next_to_top_pillbug(s, c));
        if (!actor) continue;
        for (int dt = 0; dt < NDIR; dt++) { /* summarize_pillbug_throws_for_fnn :1379-1410 */
            int t = NB[c][dt];
            uint16_t drops[NDIR];
            if (throw_drops(s, &k, c, t, drops) > 0) flag_move(s, out, &n, &seen, top_type(s, t), t);
        }
    }
    if (n == 0) { put_move(out, 0, MV_PASS, 0, 0, 0); return 1; }
    return n;
}

/* has_queen_escape_move :771-821 */
static int queen_escape(const hstate* s) {
    int me = side_to_move(s);
    if (!queen_down(s, me)) return 0;
    int q = s->queen[me];
    if (q >= NCELL || !occ_at(s, q)) return 0;
    pos_cache k;
    cache_init(s, &k);
    uint16_t tmp[NDIR];
    if (top_type(s, q) == PT_Q && top_color(s, q) == me && !bget(k.pinned, q) && dests_step(s, q, tmp) > 0)
        return 1;
    const uint64_t* mine = me ? s->btop : s->wtop;
    FOR_EACH_BIT(mine, c) {
        int pt = top_type(s, c);
        int actor = (pt == PT_P) || (pt == PT_M && s->height[c] == 1 && next_to_top_pillbug(s, c));
        if (!actor || dir_between(c, q) < 0) continue;
        if (throw_drops(s, &k, c, q, tmp) > 0) return 1;
    }
    return 0;
}

/* ---- FNN features: fnn_features.cuh:44-61 (hex_distance), :68-331 ---- */
static int hexdist(int a, int b) {
    int dq = (b % GRID) - (a % GRID), dr = (b / GRID) - (a / GRID), ds = -(dq + dr);
    int m = abs(dq);
    if (abs(dr) > m) m = abs(dr);
    if (abs(ds) > m) m = abs(ds);
    return m;
}

static void fnn_features(const hstate* s, const hmove* mv, int nmv, float* f) {
    for (int i = 0; i < OR_FEAT_DIM; i++) f[i] = 0.0f;
    float dsum[2][8] = {{0}};
    int dcnt[2][8] = {{0}};
    int ring[2] = {0, 0};
    uint64_t ap[NWORD];
    articulation(s, ap);
    int pbc[2][8], npb[2] = {0, 0};
    for (int c = 0; c < NCELL; c++) {
        int h = s->height[c];
        if (!h) continue;
        uint8_t top = s->stack[h - 1][c];
        int pt = top & 15, col = (top >> 4) & 1, tc = (pt - 1) * 2 + col;
        f[tc] += 1.0f;
        int nocc = 0;
        for (int d = 0; d < NDIR; d++) {
            int nb = NB[c][d];
            if (nb >= 0 && s->height[nb] > 0) nocc++;
        }
        if (nocc == 0) f[96 + col] += 1.0f;
        uint16_t oq = s->queen[col ^ 1];
        if (oq != 0xFFFF) {
            for (int d = 0; d < NDIR; d++)
                if (NB[c][d] >= 0 && (uint16_t)NB[c][d] == oq) { f[32 + tc] += 1.0f; break; }
        }
        for (int qc = 0; qc < 2; qc++) {
            uint16_t qcell = s->queen[qc];
            if (qcell == 0xFFFF) continue;
            for (int d = 0; d < NDIR; d++)
                if (NB[qcell][d] >= 0 && (uint16_t)NB[qcell][d] == (uint16_t)c) { ring[qc]++; break; }
        }
        if (oq != 0xFFFF) {
            dsum[col][pt - 1] += (float)hexdist(c, oq);
            dcnt[col][pt - 1] += 1;
        }
        if (h == 1 && bget(ap, c)) f[80 + tc] += 1.0f;
        if (pt != PT_Q) {
            for (int lv = 0; lv < h - 1; lv++) {
                uint8_t b = s->stack[lv][c];
                if ((b & 15) == PT_Q) f[98 + ((b >> 4) & 1)] = 1.0f;
            }
        }
        int capable = (s->stun != (uint16_t)c) && pt == PT_P;
        if (!capable && s->stun != (uint16_t)c && pt == PT_M && h == 1) {
            for (int d = 0; d < NDIR; d++) {
                int nb = NB[c][d];
                if (nb < 0 || s->height[nb] == 0 || s->stun == (uint16_t)nb) continue;
                if (top_type(s, nb) == PT_P) { capable = 1; break; }
            }
        }
        if (capable) {
            f[104 + col] = 1.0f;
            if (npb[col] < 8) pbc[col][npb[col]++] = c;
        }
    }
    for (int col = 0; col < 2; col++)
        for (int t = 0; t < 8; t++)
            if (dcnt[col][t] > 0) f[48 + t * 2 + col] = dsum[col][t] / (float)dcnt[col][t] / 10.0f;
    for (int col = 0; col < 2; col++)
        for (int t = 0; t < 8; t++) f[16 + t * 2 + col] = (float)s->hand[col][t] / (float)PER_TYPE[t];
    /* legal-move features */
    uint64_t froms[16][NWORD];
    memset(froms, 0, sizeof(froms));
    uint64_t places[NWORD] = {0};
    int me = side_to_move(s);
    for (int i = 0; i < nmv; i++) {
        if (mv[i].type == MV_MOVE) {
            int owner = me, h = s->height[mv[i].from];
            if (h > 0) owner = (s->stack[h - 1][mv[i].from] >> 4) & 1;
            bset(froms[(mv[i].pt - 1) * 2 + owner], mv[i].from);
        } else if (mv[i].type == MV_PLACE) {
            bset(places, mv[i].to);
        }
    }
    for (int i = 0; i < 16; i++) f[64 + i] = (float)bpop(froms[i]);
    f[100 + me] = (float)bpop(places) / 10.0f;
    int left = 200 - (int)s->turn;
    if (left < 0) left = 0;
    f[102] = (float)left / 200.0f;
    float t = (float)s->turn / 100.0f;
    f[103] = t < 1.0f ? t : 1.0f;
    for (int col = 0; col < 2; col++) {
        for (int i = 0; i < npb[col]; i++) {
            int p = pbc[col][i];
            for (int d = 0; d < NDIR; d++) {
                int nb = NB[p][d];
                if (nb < 0 || s->height[nb] == 0 || s->stun == (uint16_t)nb) continue;
                int nc = top_color(s, nb);
                if (nc == col) f[106 + col] += 1.0f;
                else f[108 + nc] += 1.0f;
            }
        }
    }
    for (int qc = 0; qc < 2; qc++)
        if (ring[qc] >= 1 && ring[qc] <= 6) f[110 + qc * 6 + ring[qc] - 1] = 1.0f;
}

/* ---- centroid + action index ---- */
static int round_half_even_div(int sum, int n) { /* bankers_round_div state_encoder.cuh:55-79 */
    int q = sum / n, r = sum - q * n;
    int twice = 2 * r < 0 ? -2 * r : 2 * r;
    int away = sum > 0 ? q + 1 : q - 1;
    if (twice > n) return away;
    if (twice < n) return q;
    return (q & 1) == 0 ? q : away;
}

static void centroid(const hstate* s, int* cq, int* cr) { /* compute_centroid state_encoder.cuh:889-906 */
    int sq = 0, sr = 0, n = 0;
    for (int c = 0; c < NCELL; c++) {
        if (s->height[c] > 0) { sq += c % GRID - HALF; sr += c / GRID - HALF; n++; }
    }
    *cq = n ? round_half_even_div(sq, n) : 0;
    *cr = n ? round_half_even_div(sr, n) : 0;
}

enum { EGRID = 17, EHALF = 8, ECELLS = EGRID * EGRID, MOVE_BASE = 8 * ECELLS, PASS_INDEX = MOVE_BASE + ECELLS * ECELLS };

static int window_index(int cell, int cq, int cr) { /* -1 outside the 17x17 window */
    int ec = (cell % GRID - HALF) - cq + EHALF, er = (cell / GRID - HALF) - cr + EHALF;
    if (ec < 0 || ec >= EGRID || er < 0 || er >= EGRID) return -1;
    return er * EGRID + ec;
}

static int move_action(const hmove* m, int cq, int cr) { /* gpu_move_to_action mcts_tree.cuh:146-179 */
    if (m->type == MV_PASS) return PASS_INDEX;
    if (m->type == MV_PLACE) {
        int w = window_index(m->to, cq, cr);
        return w < 0 ? -1 : ((int)m->pt - 1) * ECELLS + w;
    }
    int a = window_index(m->from, cq, cr), b = window_index(m->to, cq, cr);
    if (a < 0 || b < 0) return -1;
    return MOVE_BASE + a * ECELLS + b;
}

/* ---- public single-state API ---- */
/* ---- root tactical probe: game_logic.cu:257-397, move_gen.cuh:825-898 ---- */
static int surround_count(const hstate* s, int colour) { /* queen_surround_count_for_color game_logic.cu:257-263 */
    if (!queen_down(s, colour)) return 0;
    return occupied_neighbours(s, s->queen[colour]);
}

static int lone_empty_neighbour(const hstate* s, int target) { /* lone_empty_neighbor_of_queen move_gen.cuh:833-851 */
    if (!queen_down(s, target)) return -1;
    int q = s->queen[target];
    if (q >= NCELL) return -1;
    if (occupied_neighbours(s, q) != 5) return -1;
    int e = -1;
    for (int d = 0; d < NDIR; d++) {
        int nb = NB[q][d];
        if (nb < 0) continue;
        if (!occ_at(s, nb)) {
            if (e >= 0) return -1;
            e = nb;
        }
    }
    return e;
}

static int wins_for(int result, int colour) { return result == (colour == 0 ? RES_WHITE : RES_BLACK); }

/* has_immediate_surround_win_for_current_player, move_gen.cuh:853-874 */
static int immediate_win(const hstate* s) {
    int me = side_to_move(s);
    int cell = lone_empty_neighbour(s, me ^ 1);
    if (cell < 0) return 0;
    hmove mv[MAXLEG];
    int n = legal_moves(s, mv);
    for (int i = 0; i < n; i++) {
        if ((int)mv[i].to != cell) continue;
        hstate c = *s;
        apply(&c, &mv[i]);
        if (wins_for(c.result, me)) return 1;
    }
    return 0;
}

/* root_tactical_probe_kernel, game_logic.cu:290-397, for one root */
static void root_probe(const hstate* root, const hmove* moves, int nlegal, const float* priors, int win1,
                       int screen, int win2, int64_t* win_out, uint8_t* allowed, uint8_t* forced) {
    *win_out = -1;
    *forced = 0;
    for (int i = 0; i < MAXLEG; i++) allowed[i] = i < nlegal;
    if (nlegal <= 0 || root->result != RES_NONE) return;
    int me = side_to_move(root), opp = me ^ 1;
    int opp_s = surround_count(root, opp), own_s = surround_count(root, me);
    if (win1 && opp_s == 5) { /* 1: immediate win, best prior (first on ties) */
        int best = -1;
        float bp = -1e30f;
        for (int i = 0; i < nlegal; i++) {
            hstate c = *root;
            apply(&c, &moves[i]);
            if (wins_for(c.result, me) && (best < 0 || priors[i] > bp)) {
                best = i;
                bp = priors[i];
            }
        }
        if (best >= 0) {
            *win_out = best;
            return;
        }
    }
    if (screen && own_s == 5) { /* 2: moves after which the opponent wins at once are not allowed */
        int any_safe = 0;
        for (int i = 0; i < nlegal; i++) {
            hstate c = *root;
            apply(&c, &moves[i]);
            int bad = immediate_win(&c);
            allowed[i] = !bad;
            any_safe |= !bad;
        }
        if (!any_safe) {
            *forced = 1;
            return;
        }
    }
    if (!win2 || !(opp_s == 4 || opp_s == 5)) return;
    for (int i = 0; i < nlegal; i++) { /* 3: surround-raising moves every reply to which loses at once */
        if (!allowed[i]) continue;
        hstate c = *root;
        apply(&c, &moves[i]);
        int cs = surround_count(&c, opp);
        if (opp_s == 4 && cs <= opp_s) continue;
        if (opp_s == 5 && cs < opp_s) continue;
        hmove rep[MAXLEG];
        int nr = legal_moves(&c, rep); /* generate_non_decreasing_surround_replies move_gen.cuh:876-898 */
        int monotone = 1;
        for (int r = 0; r < nr && monotone; r++) {
            hstate g = c;
            apply(&g, &rep[r]);
            if (surround_count(&g, opp) < cs) monotone = 0;
        }
        if (!monotone) continue;
        int ok = 1;
        for (int r = 0; r < nr && ok; r++) {
            hstate g = c;
            apply(&g, &rep[r]);
            if (!wins_for(g.result, me) && !immediate_win(&g)) ok = 0;
        }
        if (ok) {
            *win_out = i;
            return;
        }
    }
}

int or_state_bytes(void) { return (int)sizeof(hstate); }

int or_legal_moves(const uint8_t* raw, uint8_t* out) {
    hmove mv[MAXLEG];
    memset(mv, 0, sizeof(mv));
    int n = legal_moves((const hstate*)raw, mv);
    memcpy(out, mv, sizeof(mv));
    return n;
}

int or_fnn_feature_moves(const uint8_t* raw, uint8_t* out) {
    hmove mv[MAXLEG + 16];
    memset(mv, 0, sizeof(mv));
    int n = compact_moves((const hstate*)raw, mv);
    memcpy(out, mv, MAXLEG * sizeof(hmove));
    return n;
}

void or_fnn_features(const uint8_t* raw, const uint8_t* moves, int n, float* f) {
    hmove mv[MAXLEG];
    if (n > MAXLEG) n = MAXLEG;
    if (n < 0) n = 0;
    memcpy(mv, moves, (size_t)n * sizeof(hmove));
    fnn_features((const hstate*)raw, mv, n, f);
}

void or_centroid(const uint8_t* raw, int* cq, int* cr) { centroid((const hstate*)raw, cq, cr); }

int or_move_to_action(const uint8_t* mv6, int cq, int cr) {
    hmove m;
    memcpy(&m, mv6, sizeof(m));
    return move_action(&m, cq, cr);
}

int or_queen_escape(const uint8_t* raw) { return queen_escape((const hstate*)raw); }

void or_neighbor_table(int16_t* out) { memcpy(out, NB, sizeof(NB)); }

/* ---- batched helpers with a static partition over pthreads ---- */
typedef struct {
    int64_t lo, hi;
    void* ctx;
    void (*body)(int64_t, void*);
} span_t;

static void* span_run(void* p) {
    span_t* sp = (span_t*)p;
    for (int64_t i = sp->lo; i < sp->hi; i++) sp->body(i, sp->ctx);
    return NULL;
}

static void parallel_for(int64_t n, int threads, void (*body)(int64_t, void*), void* ctx) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    if (threads == 1 || n < 2) {
        for (int64_t i = 0; i < n; i++) body(i, ctx);
        return;
    }
    pthread_t tid[256];
    span_t sp[256];
    for (int t = 0; t < threads; t++) {
        sp[t].lo = n * t / threads;
        sp[t].hi = n * (t + 1) / threads;
        sp[t].ctx = ctx;
        sp[t].body = body;
        pthread_create(&tid[t], NULL, span_run, &sp[t]);
    }
    for (int t = 0; t < threads; t++) pthread_join(tid[t], NULL);
}

typedef struct {
    const uint8_t* states;
    uint8_t* moves;
    int32_t* n;
    float* feat;
    int32_t* act;
} lfa_ctx;

static void lfa_body(int64_t i, void* p) {
    lfa_ctx* c = (lfa_ctx*)p;
    const hstate* s = (const hstate*)(c->states + i * OR_STATE_BYTES);
    hmove mv[MAXLEG];
    memset(mv, 0, sizeof(mv));
    int n = legal_moves(s, mv);
    if (c->moves) memcpy(c->moves + i * MAXLEG * OR_MOVE_BYTES, mv, sizeof(mv));
    if (c->n) c->n[i] = n;
    if (c->feat) fnn_features(s, mv, n, c->feat + i * OR_FEAT_DIM);
    if (c->act) {
        int cq, cr;
        centroid(s, &cq, &cr);
        int32_t* a = c->act + i * MAXLEG;
        for (int m = 0; m < MAXLEG; m++) a[m] = m < n ? move_action(&mv[m], cq, cr) : -1;
    }
}

void or_batch_legal_features_actions(const uint8_t* states, int64_t B, uint8_t* moves_out,
                                     int32_t* n_out, float* feat_out, int32_t* act_out, int threads) {
    lfa_ctx c = {states, moves_out, n_out, feat_out, act_out};
    parallel_for(B, threads, lfa_body, &c);
}

typedef struct {
    const uint8_t* states;
    const uint8_t* legal;
    const int64_t* root;
    const int64_t* idx;
    float* feat;
    int full;
} succ_ctx;

static void succ_body(int64_t i, void* p) {
    succ_ctx* c = (succ_ctx*)p;
    hstate child;
    memcpy(&child, c->states + c->root[i] * OR_STATE_BYTES, sizeof(child));
    hmove m;
    memcpy(&m, c->legal + (c->root[i] * MAXLEG + c->idx[i]) * OR_MOVE_BYTES, sizeof(m));
    apply(&child, &m);
    hmove mv[MAXLEG + 16];
    int n = c->full ? legal_moves(&child, mv) : compact_moves(&child, mv);
    fnn_features(&child, mv, n, c->feat + i * OR_FEAT_DIM);
}

void or_batch_successor_features(const uint8_t* states, const uint8_t* legal, const int64_t* action_to_root,
                                 const int64_t* move_indices, int64_t N, float* feat_out, int full_list,
                                 int threads) {
    succ_ctx c = {states, legal, action_to_root, move_indices, feat_out, full_list};
    parallel_for(N, threads, succ_body, &c);
}

typedef struct {
    const uint8_t* states;
    uint8_t* out;
} qe_ctx;

static void qe_body(int64_t i, void* p) {
    qe_ctx* c = (qe_ctx*)p;
    c->out[i] = (uint8_t)queen_escape((const hstate*)(c->states + i * OR_STATE_BYTES));
}

void or_batch_queen_escape(const uint8_t* states, int64_t B, uint8_t* out, int threads) {
    qe_ctx c = {states, out};
    parallel_for(B, threads, qe_body, &c);
}

/* ---- Philox4x32-10 (Salmon et al., SC'11, "Parallel random numbers: as easy
 * as 1, 2, 3"), multipliers 0xD2511F53 / 0xCD9E8D57, Weyl keys
 * 0x9E3779B9 / 0xBB67AE85. ---- */
/* legal_mask_kernel (state_encoder.cuh:908-976): masks [B, 85834] zero-filled by the caller */
void or_legal_mask(const uint8_t* states, const uint8_t* legal, const int32_t* nlegal, int64_t B, float* masks) {
    for (int64_t i = 0; i < B; i++) {
        int cq, cr;
        centroid((const hstate*)(states + i * OR_STATE_BYTES), &cq, &cr);
        for (int m = 0; m < nlegal[i] && m < MAXLEG; m++) {
            hmove mv;
            memcpy(&mv, legal + (i * MAXLEG + m) * OR_MOVE_BYTES, sizeof(mv));
            int a = move_action(&mv, cq, cr);
            if (a >= 0) masks[i * 85834 + a] = 1.0f;
        }
    }
}

typedef struct {
    const uint8_t* states;
    const uint8_t* legal;
    const int32_t* nlegal;
    const float* priors;
    int f1, f2, f3;
    int64_t* win;
    uint8_t* allowed;
    uint8_t* forced;
} probe_ctx;

static void probe_body(int64_t i, void* p) {
    probe_ctx* c = (probe_ctx*)p;
    hmove mv[MAXLEG];
    memcpy(mv, c->legal + i * MAXLEG * OR_MOVE_BYTES, sizeof(mv));
    root_probe((const hstate*)(c->states + i * OR_STATE_BYTES), mv, c->nlegal[i], c->priors + i * MAXLEG, c->f1,
               c->f2, c->f3, c->win + i, c->allowed + i * MAXLEG, c->forced + i);
}

void or_batch_root_tactical_probe(const uint8_t* states, const uint8_t* legal, const int32_t* nlegal,
                                  const float* priors, int64_t B, int win1, int screen, int win2, int64_t* win,
                                  uint8_t* allowed, uint8_t* forced, int threads) {
    probe_ctx c = {states, legal, nlegal, priors, win1, screen, win2, win, allowed, forced};
    parallel_for(B, threads, probe_body, &c);
}

int or_surround_count(const uint8_t* raw, int colour) { return surround_count((const hstate*)raw, colour); }
int or_immediate_win(const uint8_t* raw) { return immediate_win((const hstate*)raw); }

void or_philox4x32_10(uint32_t k0, uint32_t k1, const uint32_t ctr[4], uint32_t out[4]) {
    uint32_t x0 = ctr[0], x1 = ctr[1], x2 = ctr[2], x3 = ctr[3];
    for (int r = 0; r < 10; r++) {
        uint64_t p0 = (uint64_t)0xD2511F53u * x0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * x2;
        uint32_t y0 = (uint32_t)(p1 >> 32) ^ x1 ^ k0;
        uint32_t y1 = (uint32_t)p1;
        uint32_t y2 = (uint32_t)(p0 >> 32) ^ x3 ^ k1;
        uint32_t y3 = (uint32_t)p0;
        x0 = y0; x1 = y1; x2 = y2; x3 = y3;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = x0; out[1] = x1; out[2] = x2; out[3] = x3;
}

/* Position i: ply = philox(seed, (i,0,0,0))[0] mod (max_ply+1) (or max_ply
 * itself in lockstep mode); then for p < ply while in progress:
 * idx = (philox(seed, (i,p+1,0,0))[0] * n_legal) >> 32 and apply legal[idx]. */
typedef struct {
    uint8_t* states;
    int32_t* plies;
    int mask, max_ply, lockstep;
    uint32_t seed;
} gen_ctx;

static void gen_body(int64_t i, void* p) {
    gen_ctx* c = (gen_ctx*)p;
    hstate* s = (hstate*)(c->states + i * OR_STATE_BYTES);
    or_init_state((uint8_t*)s, c->mask);
    uint32_t ctr[4] = {(uint32_t)i, 0, 0, 0}, r[4];
    int plies;
    if (c->lockstep) {
        plies = c->max_ply;
    } else {
        or_philox4x32_10(c->seed, 0, ctr, r);
        plies = (int)(r[0] % (uint32_t)(c->max_ply + 1));
    }
    int done = 0;
    hmove mv[MAXLEG];
    for (int ply = 0; ply < plies && s->result == RES_NONE; ply++) {
        int n = legal_moves(s, mv);
        ctr[1] = (uint32_t)(ply + 1);
        or_philox4x32_10(c->seed, 0, ctr, r);
        int pick = (int)(((uint64_t)r[0] * (uint64_t)n) >> 32);
        apply(s, &mv[pick]);
        done++;
    }
    if (c->plies) c->plies[i] = done;
}

void or_generate_positions(int64_t B, int mask, int max_ply, uint32_t seed, uint8_t* states_out,
                           int32_t* plies_out, int threads) {
    gen_ctx c = {states_out, plies_out, mask, max_ply, 0, seed};
    parallel_for(B, threads, gen_body, &c);
}

void or_lockstep_selfplay(int64_t G, int mask, int max_ply, uint32_t seed, uint8_t* states_out,
                          int32_t* plies_out, int threads) {
    gen_ctx c = {states_out, plies_out, mask, max_ply, 1, seed};
    parallel_for(G, threads, gen_body, &c);
}
