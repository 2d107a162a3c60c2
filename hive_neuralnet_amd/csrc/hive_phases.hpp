// hive_phases.hpp -- the per-position phases built on hive_wave.hpp:
// legal-list generation and assembly, FNN features, action indices,
// compact successor summaries and move application on the LDS board.
#pragma once

#include "hive_wave.hpp"

namespace hw {

// ---------------------------------------------------------------- legal list
// generate_legal_moves (move_gen.cuh:1151-1360): placements (cells ascending
// x placeable types), then moves of each own top piece that is neither
// stunned nor pinned (cells ascending, type-specific order), then pillbug
// throws (own top pillbugs, then own ground mosquitoes touching a top
// pillbug, in cell order), cut at 256; a lone PASS when empty; nothing when
// the game is over.
//
// The list is not materialised in LDS: generate_legal leaves the placement
// cells (P.plc, P.plc_pre), the per-piece destination lists (P.u2.pool), the
// throw lists and the segment starts (P.seg_base: placements, one segment
// per piece, one per throw actor, end) on the board; list_slot() decodes any
// slot from them, so that slots are written to memory lane-parallel.
struct ListInfo {
    int n;          // list length after the cut (1 for a lone PASS, 0 when the game is over)
    int total;      // entries before the cut
    int n_place;    // placement entries (npos * ntypes)
    int npos;       // placement cells
    int ntypes;     // placeable types emitted per cell
    int n_pieces;   // piece segments
    int nseg;       // segments before the end marker
    uint32_t emit_types;
    uint32_t type_list;  // the emitted placeable types, ascending, one per nibble
    int ub_total;        // gated lists: a bound on the whole list's length (the full list: total)
};

// Which pieces generate_legal runs.  The full list runs every piece.  A gate
// with kTargeted set may skip a piece (its segment is then empty) and may
// stop the ant searches once they reach cell `stop`; generate_legal then
// reports in ub_total a bound on the length of the whole list, with each
// skipped or stopped piece counted at the most destinations it can have.
struct FullList {
    static constexpr bool kTargeted = false;
    int stop = -1;
    HW_INL bool run(const Pos&, int, int) const { return true; }
};

// The most destinations a piece of type t can have on a board whose hive has
// e empty neighbour cells: sliding searches end on such cells (an ant or a
// spider can end on no other; the origin is never one), the others have
// their generators' bounds.
__device__ __forceinline__ int dest_bound(int t, int e) {
    switch (t) {
        case PT_A: return min(e, kAntCap);
        case PT_S: return min(e, 32);
        case PT_L: return 32;
        case PT_M: return 64;
        default: return 6;
    }
}

template <class Gate = FullList>
HW_INL ListInfo generate_legal(Pos& P, int lane, const Gate& G = Gate()) {
    const int l = gl(lane);
    ListInfo L{0, 0, 0, 0, 0, 0, 0, 0u, 0u, 0};
    const bool go = P.result == 0;  // barriers below are reached by both positions of the wave
    const int me = P.turn & 1;
    const int ptn = P.turn >> 1;
    const bool queen_down = (P.qplaced >> me) & 1;
    const bool queen_now = (ptn == 3) && !queen_down;
    const uint32_t held = hand_mask(P, me);
    const uint32_t placeable = go ? (queen_now ? (held & 1u) : held) : 0u;
    uint32_t emit_types = placeable & ~(ptn == 0 ? 1u : 0u);
    int ntypes = __popc(emit_types);

    // -- placement cells, lane w < 18 owns board word w
    uint32_t pw = 0;
    if (placeable && l < 18) {
        if (P.turn == 0) {
            pw = (l == (264 >> 5)) ? (1u << (264 & 31)) : 0u;
        } else if (P.turn == 1) {
            pw = nbr_union_word(P.occ, l) & ~P.occ[l + 1];
        } else {
            const uint32_t* mine = me ? P.bt : P.wt;
            const uint32_t* theirs = me ? P.wt : P.bt;
            pw = nbr_union_word(mine, l) & ~nbr_union_word(theirs, l) & ~P.occ[l + 1];
        }
    }
    int prank = grp_excl_scan(__popc(pw));
    int npos = grp_sum(__popc(pw), lane);
    if (l < 18) {
        P.plc[l + 1] = pw;
        P.plc_pre[l] = (uint16_t)prank;
    }
    int n_place = npos * ntypes;

    // -- movable pieces (own top cells, not stunned, not pinned) and throw
    // actors, both in cell order: one lane per occupied cell (the list is
    // ascending), ranks by ballot.  The thrower is not checked for stun or
    // pin (move_gen.cuh:1304-1345).
    int n_pieces = 0, n_actors = 0;
    if (go && queen_down) {
        bool movable = false, actor = false;
        int c = 0, tb = 0;
        if (l < P.n_occ) {
            c = P.occ_cells[l];
            tb = P.tp(c);
            const int t = tb & 15;
            movable = pb_get(me ? P.bt : P.wt, c) && !pb_get(P.pin, c) && c != (int)P.stun;
            if (((tb >> 4) & 1) == me)
                actor = (t == PT_P) || (t == PT_M && P.hgt(c) == 1 && touches_top_pillbug(P, c));
        }
        const uint32_t below = (1u << l) - 1u;
        const uint32_t pm = grp_ballot(movable, lane);
        n_pieces = min(__popc(pm), kMaxPieces);
        if (movable) {
            const int k = __popc(pm & below);
            if (k < kMaxPieces) {
                P.piece_cell[k] = (uint16_t)c;
                P.piece_type[k] = (uint8_t)(tb & 15);
            }
        }
        const uint32_t am = grp_ballot(actor, lane);
        n_actors = min(__popc(am), kActors);
        if (actor) {
            const int r = __popc(am & below);
            if (r < kActors) P.actor_cell[r] = (uint16_t)c;
        }
    }
    __syncthreads();

    // -- destination pool offsets by type capacity, visited sets by need;
    // lanes 0..15 run the pieces, lanes 16, 17 the throw actors
    int cap = l < n_pieces ? type_capacity(P.piece_type[l]) : 0;
    int off = grp_excl_scan(cap);
    int nsets = l < n_pieces ? type_sets(P.piece_type[l]) : 0;
    int set0 = grp_excl_scan(nsets);
    // gated lists: the empty cells next to the hive bound the sliding searches
    int empties = 0;
    if (Gate::kTargeted) {
        const uint32_t ew = l < 18 ? nbr_union_word(P.occ, l) & ~P.occ[l + 1] : 0u;
        empties = grp_sum(__popc(ew), lane);
    }
    int ub = 0;  // this lane's piece or throw actor, counted toward ub_total
    bool ant_job = false;  // an ant search left to the group (ant_searches)
    int c = 0, ant_next = 0, ant_len = 0;
    RingLift ant_rl{0, 0u, 0u};
    if (l < n_pieces && (off + cap > kPool || set0 + nsets > kSets)) {  // impossible piece counts
        P.piece_off[l] = 0;
        P.piece_cnt[l] = 0;
    } else if (l < n_pieces) {
        c = P.piece_cell[l];
        int t = P.piece_type[l];
        uint16_t* out = P.u2.pool + off;
        uint32_t* s0 = P.u1.sets[set0 < kSets ? set0 : 0];
        uint32_t* s1 = P.u1.sets[set0 + 1 < kSets ? set0 + 1 : 0];
        int m = 0;
        bool stopped = false;
        const bool run = G.run(P, c, t);
        if (run) {
            switch (t) {
                case PT_Q: case PT_P: m = gen_step(P, c, out); break;
                case PT_A:
                    if (kAntGroup) {
                        m = gen_ant<Gate::kTargeted, true>(P, c, out, kAntCap, s0, G.stop, &stopped, kAntLaneSteps,
                                                           &ant_next, &ant_rl);
                        ant_job = !stopped && ant_next < m && m < kAntCap;
                        ant_len = m;
                    } else {
                        m = gen_ant<Gate::kTargeted>(P, c, out, kAntCap, s0, G.stop, &stopped);
                    }
                    break;
                case PT_G: m = gen_hopper(P, c, out); break;
                case PT_S: m = gen_spider(P, c, out, s0); break;
                case PT_B: m = gen_beetle(P, c, out); break;
                case PT_M: m = gen_mosquito<Gate::kTargeted>(P, c, out, s0, s1, G.stop, &stopped); break;
                case PT_L: m = gen_ladybug(P, c, out, s0); break;
                default: break;
            }
        }
        P.piece_off[l] = (uint16_t)off;
        P.piece_cnt[l] = (uint8_t)m;
        ub = (run && !stopped) ? m : dest_bound(t, empties);
    } else if (l >= kMaxPieces && l - kMaxPieces < n_actors) {
        int j = l - kMaxPieces;
        P.throw_cnt[j] = (uint16_t)gen_throws(P, P.actor_cell[j], P.throw_from[j], P.throw_to[j], P.throw_pt[j]);
        ub = P.throw_cnt[j];
    }
    if (kAntGroup) {
        int m = 0;
        bool stopped = false;
        ant_searches<Gate::kTargeted>(P, lane, ant_job, c, off, kAntCap, set0 < kSets ? set0 : 0, ant_len, ant_next,
                                      ant_rl, G.stop, m, stopped);
        if (ant_job) {
            P.piece_cnt[l] = (uint8_t)m;
            ub = stopped ? dest_bound(PT_A, empties) : m;
        }
    }
    if (Gate::kTargeted) L.ub_total = n_place + grp_sum(ub, lane);
    __syncthreads();

    // -- segment starts: lane 0 placements, lanes 1..n_pieces pieces, then actors, then the end
    int cnt = 0;
    if (l == 0) cnt = n_place;
    else if (l <= n_pieces) cnt = P.piece_cnt[l - 1];
    else if (l <= n_pieces + n_actors) cnt = P.throw_cnt[l - 1 - n_pieces];
    int base = grp_excl_scan(cnt);
    int total = grp_sum(cnt, lane);
    int nseg = 1 + n_pieces + n_actors;
    static_assert(kSegs <= kW, "one lane per segment start");
    P.seg_base[l] = (int16_t)(l <= nseg ? min(base, 32767) : 32767);
    __syncthreads();
    if (!go) return L;
    L.total = total;
    if (!Gate::kTargeted) L.ub_total = total;
    L.n = total == 0 ? 1 : (total < kMaxLegal ? total : kMaxLegal);  // PASS = all-zero from/to, type 2
    L.n_place = n_place;
    L.npos = npos;
    L.ntypes = ntypes;
    L.n_pieces = n_pieces;
    L.nseg = nseg;
    L.emit_types = emit_types;
    for (uint32_t m = emit_types, k = 0; m; m &= m - 1, k += 4) L.type_list |= (uint32_t)__ffs(m) << k;
    return L;
}

// position of the r-th set bit of x (r < popc(x))
__device__ __forceinline__ int select_bit(uint32_t x, int r) {
    int pos = 0;
    int c = __popc(x & 0xFFFFu);
    if (r >= c) { r -= c; x >>= 16; pos += 16; }
    c = __popc(x & 0xFFu);
    if (r >= c) { r -= c; x >>= 8; pos += 8; }
    c = __popc(x & 0xFu);
    if (r >= c) { r -= c; x >>= 4; pos += 4; }
    c = __popc(x & 0x3u);
    if (r >= c) { r -= c; x >>= 2; pos += 2; }
    c = (int)(x & 1u);
    if (r >= c) pos += 1;
    return pos;
}

// Slot i (i < L.n, L.total > 0) of the generated list as (type | pt << 8, from, to).
HW_INL void list_slot(const Pos& P, const ListInfo& L, int i, int& tp, int& from, int& to, int& seg) {
    // last segment starting at or before i: five fixed halving steps over
    // the non-decreasing starts (nseg <= 19 < 32; the end marker and the
    // entries past it hold starts beyond every slot)
    static_assert(kSegs <= 32, "five steps cover the segments");
    int lo = 0;
#pragma unroll
    for (int step = 16; step > 0; step >>= 1) {
        const int mid = lo + step;
        if (P.seg_base[mid] <= i) lo = mid;
    }
    seg = lo;
    int k = i - P.seg_base[lo];
    if (lo == 0) {  // placement: cell k / ntypes, type (k % ntypes)-th of emit_types
        int r = k / L.ntypes;
        int ti = k - r * L.ntypes;
        int wl = 0, wh = 17;  // last board word whose placement prefix is <= r
        while (wl < wh) {
            int mid = (wl + wh + 1) >> 1;
            if (P.plc_pre[mid] <= r) wl = mid;
            else wh = mid - 1;
        }
        to = wl * 32 + select_bit(P.plc[wl + 1], r - P.plc_pre[wl]);
        from = 0;
        tp = MV_PLACE | (((L.type_list >> (4 * ti)) & 15u) << 8);
    } else if (lo <= L.n_pieces) {
        int j = lo - 1;
        from = P.piece_cell[j];
        to = P.u2.pool[P.piece_off[j] + k] & kCellMask;
        tp = MV_MOVE | (P.piece_type[j] << 8);
    } else {
        int j = lo - 1 - L.n_pieces;
        from = P.throw_from[j][k];
        to = P.throw_to[j][k];
        tp = MV_MOVE | (P.throw_pt[j][k] << 8);
    }
}

// ---------------------------------------------------------------- features
// extract_fnn_features_device (fnn_features.cuh:68-331).  The legal-move
// features (distinct MOVE sources per (type, owner), distinct PLACE
// destinations) come from the from_bb / place_bb sets filled while a list is
// written or read (kFeatList, kFeatGen: place count given), or, for compact
// successor lists, from a (type, owner) bucket mask and a placement count
// (kFeatBucket).  S is the state row (for the stacked levels under a top
// piece).
enum { kFeatList = 0, kFeatGen = 1, kFeatBucket = 2 };

// The list's source sets (u1: after destination generation; X: a
// caller-supplied list's cell sets) ...
HW_INL void sources_clear(Pos& P, int lane, ListSets* X = nullptr) {
    const int l = gl(lane);
    if (l < 16) P.u1.e.from_d[l] = 0;
    if (X) {
        for (int i = l; i < 16 * 18; i += kW) (&X->from_bb[0][0])[i] = 0;
        if (l < 18) X->place_bb[l] = 0;
    }
}
// ... and the feature counters (u2: after list emission).
HW_INL void counters_clear(Pos& P, int lane) {
    const int l = gl(lane);
    auto& F = P.u2.c;
    for (int i = l; i < 128; i += kW) F.cnt[i] = 0;
    if (l < 16) { F.dsum[l] = 0; F.dcnt[l] = 0; }
    if (l < 2) { F.ring[l] = 0; F.covered[l] = 0; F.capable[l] = 0; }
    if (l == 0) F.n_cap = 0;
}

// MOVE source / PLACE destination sets of a caller-supplied list (global memory)
HW_INL void list_sources(Pos& P, const uint8_t* __restrict__ M, int n, int lane, ListSets& F) {
    const int me = P.turn & 1;
    for (int i = gl(lane); i < n; i += kW) {
        const uint8_t* m = M + 6 * i;
        int ty = m[0], pt = m[1];
        if (ty == MV_MOVE) {
            int fc = m[2] | (m[3] << 8);
            if (fc < 544 && pt >= 1 && pt <= 8) {
                int owner = P.hgt(fc) > 0 ? (P.tp(fc) >> 4) & 1 : me;
                atomicOr(&F.from_bb[(pt - 1) * 2 + owner][fc >> 5], 1u << (fc & 31));
            }
        } else if (ty == MV_PLACE) {
            int tc = m[4] | (m[5] << 8);
            if (tc < 544) atomicOr(&F.place_bb[tc >> 5], 1u << (tc & 31));
        }
    }
}

// x / d rounded as IEEE division rounds it, for the features' divisors:
// q = x * rd with rd = 1 / d rounded to float, then one residual step
// q + fma(-q, d, x) * rd.  It gives the correctly rounded quotient for every
// integer x in [0, 2^24) with d in {3, 10, 100, 200}, and for (s / n) / 10
// with n <= 3, s < 4096 (both checked exhaustively against host division
// under the wave emulator); with d = 1 or 2 every step is exact.  A quarter of
// the instructions of the full division sequence.
__device__ __forceinline__ float div_exact(float x, float d, float rd) {
    const float q = x * rd;
    return __builtin_fmaf(__builtin_fmaf(-q, d, x), rd, q);
}

// Needs sources_clear / counters_clear and the legal-move sets (modes kFeatList / kFeatGen)
// complete, behind a barrier.
HW_INL void features_finish(Pos& P, const uint8_t* __restrict__ S, float* __restrict__ out, int lane, int mode,
                            uint32_t bucket, int n_place, const ListSets* X = nullptr) {
    const int l = gl(lane);
    auto& F = P.u2.c;
    const int me = P.turn & 1;
    if (l < P.n_occ) {
        int c = P.occ_cells[l];
        int h = P.hgt(c);
        int tb = P.tp(c);
        int pt = tb & 15, col = (tb >> 4) & 1, tc = (pt - 1) * 2 + col;
        if (pt < PT_Q || pt > PT_P) pt = 0;  // impossible top byte: contributes nothing
        if (pt) atomicAdd(&F.cnt[tc], 1);
        uint32_t nm = P.nbd[l];
        if (nm == 0) atomicAdd(&F.cnt[96 + col], 1);
        // hex distances to both queens (hexdist, fnn_features.cuh:44-61) from c's row and column;
        // a queen on the board is c's neighbour exactly when the distance is 1
        const int rc = row_of(c), cc = c - rc * kGrid;
        auto dist_to = [&](int q) {
            const int rq = row_of(q), dq = (q - rq * kGrid) - cc, dr = rq - rc, ds = -(dq + dr);
            return max(max(abs(dq), abs(dr)), abs(ds));
        };
        const int q0 = P.queen[0], q1 = P.queen[1];
        const int d0 = q0 != 0xFFFF ? dist_to(q0) : 0, d1 = q1 != 0xFFFF ? dist_to(q1) : 0;
        const int oq = col ? q0 : q1, dopp = col ? d0 : d1;  // the opponent's queen, queen[col ^ 1]
        if (oq != 0xFFFF && pt) {
            if (oq < kCells && dopp == 1) atomicAdd(&F.cnt[32 + tc], 1);
            atomicAdd(&F.dsum[(pt - 1) * 2 + col], dopp);
            atomicAdd(&F.dcnt[(pt - 1) * 2 + col], 1);
        }
        if (q0 != 0xFFFF && q0 < kCells && d0 == 1) atomicAdd(&F.ring[0], 1);
        if (q1 != 0xFFFF && q1 < kCells && d1 == 1) atomicAdd(&F.ring[1], 1);
        if (pt && pb_get(P.pin, c)) atomicAdd(&F.cnt[80 + tc], 1);  // articulation point, one piece high
        if (pt != PT_Q && h >= 2) {
            for (int lv = 0; lv < h - 1 && lv < 5; lv++) {
                int b = S[lv * kCells + c];
                if ((b & 15) == PT_Q) F.covered[(b >> 4) & 1] = 1;
            }
        }
        bool capable = ((int)P.stun != c) && pt == PT_P;
        if (!capable && (int)P.stun != c && pt == PT_M && h == 1) {
            uint32_t m = nm;
            while (m) {
                int d = __ffs(m) - 1;
                m &= m - 1;
                int nb = step(c, d);
                if ((int)P.stun == nb) continue;
                if ((P.tp(nb) & 15) == PT_P) { capable = true; break; }
            }
        }
        if (capable) {
            F.capable[col] = 1;
            int k = atomicAdd(&F.n_cap, 1);
            if (k < 8) { F.cap_cells[k] = (uint16_t)c; F.cap_col[k] = (uint8_t)col; }
        }
    }
    __syncthreads();
    // pieces next to a pillbug-capable cell (throwable own / threatened)
    int ncap = F.n_cap < 8 ? F.n_cap : 8;
    if (l < ncap) {
        int p = F.cap_cells[l], col = F.cap_col[l];
        uint32_t m = nbo(P, p);
        while (m) {
            int d = __ffs(m) - 1;
            m &= m - 1;
            int nb = step(p, d);
            if ((int)P.stun == nb) continue;
            int nc = (P.tp(nb) >> 4) & 1;
            if (nc == col) atomicAdd(&F.cnt[106 + col], 1);
            else atomicAdd(&F.cnt[108 + nc], 1);
        }
    }
    if (mode == kFeatBucket) {
        if (l < 16) F.cnt[64 + l] = (bucket >> l) & 1u;
        else if (l == 16) F.cnt[100] = n_place;
    } else if (mode == kFeatList) {
        if (l < 16) {
            int s = 0;
            for (int w = 0; w < 18; w++) s += __popc(X->from_bb[l][w]);
            F.cnt[64 + l] = s;
        } else if (l == 16) {
            int s = 0;
            for (int w = 0; w < 18; w++) s += __popc(X->place_bb[w]);
            F.cnt[100] = s;
        }
    } else if (l < 16) {
        F.cnt[64 + l] = __popc(P.u1.e.from_d[l]);
    } else if (l == 16) {
        F.cnt[100] = n_place;
    }
    __syncthreads();
    // write-out: lane l takes features l, 32 + l, 64 + l and 96 + l, so each
    // of the four stores has only the cases of its own range
    static_assert(kW == 32 && kFeat == 122, "feature ranges per lane");
    if (!out) return;
    constexpr float kPer[8] = {1.f, 3.f, 3.f, 2.f, 2.f, 1.f, 1.f, 1.f};
    constexpr float kRcpPer[8] = {1.f, 1.f / 3.f, 1.f / 3.f, 0.5f, 0.5f, 1.f, 1.f, 1.f};
    if (l < 16) {
        out[l] = (float)F.cnt[l];
    } else {
        int t = (l - 16) >> 1, c = (l - 16) & 1;
        out[l] = div_exact((float)P.hand[c][t], kPer[t], kRcpPer[t]);
    }
    if (l < 16) {
        out[32 + l] = (float)F.cnt[32 + l];
    } else {
        // dcnt is a piece count of one type and colour, 1..3 when positive
        int k = l - 16, n = F.dcnt[k];
        const float rn = n == 3 ? 1.f / 3.f : n == 2 ? 0.5f : 1.f;
        out[32 + l] = n > 0 ? div_exact(div_exact((float)F.dsum[k], (float)n, rn), 10.0f, 0.1f) : 0.0f;
    }
    out[64 + l] = (float)F.cnt[64 + l];
    if (l < kFeat - 96) {
        int i = 96 + l;
        float v;
        if (i < 98) v = (float)F.cnt[i];
        else if (i < 100) v = F.covered[i - 98] ? 1.0f : 0.0f;
        else if (i < 102) v = (i - 100) == me ? div_exact((float)F.cnt[100], 10.0f, 0.1f) : 0.0f;
        else if (i == 102) { int left = 200 - (int)P.turn; v = div_exact((float)(left < 0 ? 0 : left), 200.0f, 0.005f); }
        else if (i == 103) { float t = div_exact((float)P.turn, 100.0f, 0.01f); v = t < 1.0f ? t : 1.0f; }
        else if (i < 106) v = F.capable[i - 104] ? 1.0f : 0.0f;
        else if (i < 110) v = (float)F.cnt[i];
        else {
            int qc = (i - 110) / 6, b = (i - 110) % 6;
            v = (F.ring[qc] == b + 1) ? 1.0f : 0.0f;
        }
        out[i] = v;
    }
}

// ---------------------------------------------------------------- actions
// bankers_round_div (state_encoder.cuh:55-79)
__device__ __forceinline__ int round_half_even_div(int sum, int n) {
    int q = sum / n, r = sum - q * n;
    int twice = abs(2 * r);
    int away = sum > 0 ? q + 1 : q - 1;
    if (twice > n) return away;
    if (twice < n) return q;
    return (q & 1) == 0 ? q : away;
}

// The same for |sum| <= 4096 and 1 <= n <= 64 (the occupied-cell list: |sum|
// <= 32 * 11, n <= 32) without an integer division.
// rcp_n is 1 / n to within 1 ulp, so f = sum * rcp_n is within 2^-10 of
// x = sum / n.  Unless x is a half-integer it is at least 1 / (2n) >= 2^-7
// from one, so rounding f to the nearest integer gives round(x); q is then
// exact and d = 2 sum - 2 q n = 2n (x - q) tells an exact tie (|d| == n),
// which goes to the even one of q and q + sign(d).
__device__ __forceinline__ int round_half_even_div(int sum, int n, float rcp_n) {
    const int q = (int)__builtin_rintf((float)sum * rcp_n);
    const int d = 2 * (sum - q * n);
    if (d == n || d == -n) return (q & 1) ? q + (d > 0 ? 1 : -1) : q;
    return q;
}

// compute_centroid (state_encoder.cuh:889-906) over the occupied-cell list
HW_INL void centroid(const Pos& P, int lane, int& cq, int& cr) {
    const int l = gl(lane);
    int q = 0, r = 0;
    if (l < P.n_occ) {
        int c = P.occ_cells[l];
        int row = row_of(c);
        q = c - row * kGrid - kHalf;
        r = row - kHalf;
    }
    int sq = grp_sum(q, lane), sr = grp_sum(r, lane), n = P.n_occ;
    const float rcp_n = __builtin_amdgcn_rcpf((float)(n ? n : 1));
    cq = n ? round_half_even_div(sq, n, rcp_n) : 0;
    cr = n ? round_half_even_div(sr, n, rcp_n) : 0;
}

__device__ __forceinline__ int window17(int cell, int cq, int cr) {
    int row = row_of(cell);
    int ec = (cell - row * kGrid - kHalf) - cq + 8, er = (row - kHalf) - cr + 8;
    return (ec < 0 || ec >= 17 || er < 0 || er >= 17) ? -1 : er * 17 + ec;
}

// gpu_move_to_action (mcts_tree.cuh:146-179), ENC_GRID = 17 -> 85,834 actions
__device__ __forceinline__ int move_action(int type, int pt, int from, int to, int cq, int cr) {
    if (type == MV_PASS) return 85833;
    if (type == MV_PLACE) {
        int w = window17(to, cq, cr);
        return w < 0 ? -1 : (pt - 1) * 289 + w;
    }
    int a = window17(from, cq, cr), b = window17(to, cq, cr);
    return (a < 0 || b < 0) ? -1 : 2312 + a * 289 + b;
}

// action indices of a caller-supplied list (global memory), -1 padded
HW_INL void list_actions(const uint8_t* __restrict__ M, int n, int cq, int cr, int* __restrict__ out, int lane) {
    for (int i = gl(lane); i < kMaxLegal; i += kW) {
        int a = -1;
        if (i < n) {
            const uint8_t* m = M + 6 * i;
            a = move_action(m[0], m[1], m[2] | (m[3] << 8), m[4] | (m[5] << 8), cq, cr);
        }
        out[i] = a;
    }
}

// Placement cells in ascending order (the first kPlist) into u1.e.plist, for
// emit_list; lane w < 18 takes board word w.  After generation (u1 no longer
// holds visited sets), before the barrier that precedes emit_list.
HW_INL void place_list(Pos& P, int lane) {
    const int l = gl(lane);
    if (l < 18) {
        uint32_t pw = P.plc[l + 1];
        int k = P.plc_pre[l];
        while (pw && k < kPlist) {
            P.u1.e.plist[k++] = (uint16_t)(32 * l + __ffs(pw) - 1);
            pw &= pw - 1;
        }
    }
}

// Writes the generated list: moves (zero padded), action indices (-1
// padded), and the MOVE-source sets of the features (one bit per piece
// segment that is inside the cut, one per throw entry), the latter one lane
// per segment before the slots.  Placement slot i is cell i / ntypes of the
// placement list with the (i % ntypes)-th placeable type (the quotient by a
// multiply: (i * ceil(65536 / ntypes)) >> 16 is exact for i < 256, ntypes
// <= 8); later slots are decoded by list_slot.  A piece's action window
// index comes from P.piece_win (set after the centroid, behind a barrier).
template <bool WithMoves, bool WithAct, bool WithFeat>
HW_INL void emit_list(Pos& P, const ListInfo& L, int lane, uint8_t* __restrict__ moves_row,
                      int32_t* __restrict__ act_row, int cq, int cr, bool pad = true) {
    const int me = P.turn & 1;
    const int l = gl(lane);
    if (WithFeat && L.total > 0) {
        const int s = l + 1;  // segment s: piece s - 1, or throw actor s - 1 - n_pieces
        if (s <= L.n_pieces) {
            const int j = s - 1;
            const int c = P.piece_cell[j], pt = P.piece_type[j];
            if (P.piece_cnt[j] > 0 && P.seg_base[s] < L.n && c < kCells && pt >= 1 && pt <= 8) {
                const int r = occ_rank(P, c);  // sources of generated moves are occupied
                if (r < 32) atomicOr(&P.u1.e.from_d[(pt - 1) * 2 + me], 1u << r);
            }
        } else if (s < L.nseg) {
            const int j = s - 1 - L.n_pieces, base = P.seg_base[s];
            for (int k = 0; k < (int)P.throw_cnt[j] && base + k < L.n; k++) {
                const int c = P.throw_from[j][k], pt = P.throw_pt[j][k];
                if (c < kCells && pt >= 1 && pt <= 8) {
                    const int r = occ_rank(P, c);
                    if (r < 32) atomicOr(&P.u1.e.from_d[(pt - 1) * 2 + ((P.tp(c) >> 4) & 1)], 1u << r);
                }
            }
        }
    }
    uint16_t* row16 = reinterpret_cast<uint16_t*>(moves_row);
    const uint32_t nt = (uint32_t)(L.ntypes > 0 ? L.ntypes : 1);
    const uint32_t inv = (65536u + nt - 1u) / nt;
    for (int i = l; i < L.n; i += kW) {
        int tp = 0, from = 0, to = 0, wfrom = 0;  // wfrom: window index of a MOVE's source
        if (L.total == 0) {
            tp = MV_PASS;
        } else if (i < L.n_place && i < kPlist) {  // cell rank <= i
            const int r = (int)(((uint32_t)i * inv) >> 16);
            to = P.u1.e.plist[r];
            tp = MV_PLACE | (((L.type_list >> (4 * (i - r * (int)nt))) & 15u) << 8);
        } else {
            int seg;
            list_slot(P, L, i, tp, from, to, seg);
            if (WithAct) {
                if (seg > L.n_pieces) wfrom = window17(from, cq, cr);  // throws
                else if (seg > 0) wfrom = P.piece_win[seg - 1];
            }
        }
        if (WithMoves) {
            row16[3 * i] = (uint16_t)tp;
            row16[3 * i + 1] = (uint16_t)from;
            row16[3 * i + 2] = (uint16_t)to;
        }
        if (WithAct) {  // gpu_move_to_action (mcts_tree.cuh:146-179) with the source's window given
            const int type = tp & 0xFF;
            int a = 85833;
            if (type != MV_PASS) {
                const int b = window17(to, cq, cr);
                if (type == MV_PLACE) a = b < 0 ? -1 : ((tp >> 8) - 1) * 289 + b;
                else a = (wfrom < 0 || b < 0) ? -1 : 2312 + wfrom * 289 + b;
            }
            act_row[i] = a;
        }
    }
    // the rest of the rows: zero moves and -1 action indices, in 16-byte stores
    // (rows are 16-byte aligned: 1,536 and 1,024 bytes per position); without
    // `pad` the rows end at the list's length
    if (!pad) return;
    if (WithMoves) {
        const int h0 = 3 * L.n, c0 = (h0 + 7) >> 3;  // first padding half-word, first whole 16-byte chunk
        if (l < 8 * c0 - h0) row16[h0 + l] = 0;
        const u32x4 z = {0u, 0u, 0u, 0u};
        for (int k = c0 + l; k < kMaxLegal * 6 / 16; k += kW) reinterpret_cast<u32x4*>(moves_row)[k] = z;
    }
    if (WithAct) {
        const int c0 = (L.n + 3) >> 2;
        if (l < 4 * c0 - L.n) act_row[L.n + l] = -1;
        const u32x4 m1 = {~0u, ~0u, ~0u, ~0u};
        for (int k = c0 + l; k < kMaxLegal / 4; k += kW) reinterpret_cast<u32x4*>(act_row)[k] = m1;
    }
}

// ---------------------------------------------------------------- summaries
// Existence predicates: "the generator for this piece type is non-empty"
// (the reference's has_*_move helpers, move_gen.cuh:214-1049).
HW_INL bool has_hopper(const Pos& P, int c) {
    uint32_t m = nbo(P, c);
    const int r0 = row_of(c), q0 = c - r0 * kGrid;
    while (m) {
        int d = __ffs(m) - 1;
        m &= m - 1;
        if (hop_dest(P, c, r0, q0, d) >= 0) return true;
    }
    return false;
}

HW_INL bool has_spider(const Pos& P, int c) {
    const Lift lf = lift_of(P, c);
    uint32_t m1 = P.sm[c];
    while (m1) {  // as gen_spider: steps back masked out
        int d1 = __ffs(m1) - 1;
        m1 &= m1 - 1;
        int p1 = c - 23 + (int)dir_byte(kOfsHi, kOfsLo, d1);
        uint32_t m2 = exits_next_to(P, p1, d1, lf) & ~dir_byte(kOppHi, kOppLo, d1);
        while (m2) {
            int d2 = __ffs(m2) - 1;
            m2 &= m2 - 1;
            int p2 = p1 - 23 + (int)dir_byte(kOfsHi, kOfsLo, d2);
            uint32_t m3 = exits_lifted(P, p2, lf) & ~dir_byte(kOppHi, kOppLo, d2);
            while (m3) {
                int d3 = __ffs(m3) - 1;
                m3 &= m3 - 1;
                if (p2 - 23 + (int)dir_byte(kOfsHi, kOfsLo, d3) != c) return true;
            }
        }
    }
    return false;
}

HW_INL bool has_beetle(const Pos& P, int c) {
    uint32_t gm = grid6(c);
    uint32_t nh = nbr_heights(P, c, gm);
    uint32_t sm = slide_mask(P, c, c);
    int below = P.hgt(c) - 1;
    for (int d = 0; d < 6; d++) {
        if (!((gm >> d) & 1u)) continue;
        int mh = max(hof(nh, d), below);
        if (mh > 0) {
            if (!gate_high(nh, d, mh)) return true;
        } else if ((sm >> d) & 1u) {
            return true;
        }
    }
    return false;
}

HW_INL bool has_ladybug(const Pos& P, int c) {
    uint32_t g0 = grid6(c);
    uint32_t nh0 = nbr_heights(P, c, g0);
    uint32_t o0 = nbo(P, c);
    int hc = P.hgt(c);
    for (int d1 = 0; d1 < 6; d1++) {
        if (!((o0 >> d1) & 1u)) continue;
        int p1 = step(c, d1);
        if (gate_high(nh0, d1, max(hc - 1, hof(nh0, d1)))) continue;
        uint32_t nh1 = nbr_heights(P, p1, grid6(p1));
        uint32_t o1 = nbo(P, p1);
        int hp1 = P.hgt(p1);
        for (int d2 = 0; d2 < 6; d2++) {
            if (!((o1 >> d2) & 1u)) continue;
            int p2 = step(p1, d2);
            if (p2 == c) continue;
            if (gate_high(nh1, d2, max(hp1, hof(nh1, d2)))) continue;
            uint32_t g2 = grid6(p2);
            uint32_t nh2 = nbr_heights(P, p2, g2);
            uint32_t o2 = nbo(P, p2);
            int mh3 = P.hgt(p2);
            for (int d3 = 0; d3 < 6; d3++) {
                if (!((g2 >> d3) & 1u) || ((o2 >> d3) & 1u)) continue;
                int p3 = step(p2, d3);
                if (p3 == c || p3 == p1) continue;
                if (!gate_high(nh2, d3, mh3)) return true;
            }
        }
    }
    return false;
}

// `climb`: the piece is one high and either has a ground-slide exit (a
// beetle's move down to the ground is that slide) or stands on a board with
// no stack and has an occupied neighbour (climbing onto a one-high neighbour
// is gated only by two flanks higher than one) -- then moving as a beetle
// succeeds, so has_beetle need not run.
// `jump`: no occupied cell on the grid's border and the piece has an occupied
// neighbour -- then a jump over it lands inside the grid (the line's last
// occupied cell lies in the hive, the landing one step beyond), so
// has_hopper need not run.
HW_INL bool piece_has_move(const Pos& P, int c, int t, bool climb = false, bool jump = false) {
    switch (t) {
        case PT_Q: case PT_P: case PT_A: return slide_mask(P, c, c) != 0;
        case PT_G: return jump || has_hopper(P, c);
        case PT_S: return has_spider(P, c);
        case PT_B: return climb || has_beetle(P, c);
        case PT_L: return has_ladybug(P, c);
        case PT_M: {
            if (P.hgt(c) > 1) return has_beetle(P, c);
            uint32_t om = nbo(P, c);
            uint32_t has = 0;
            while (om) {
                int d = __ffs(om) - 1;
                om &= om - 1;
                int tt = P.tp(step(c, d)) & 15;
                if (tt != PT_M) has |= 1u << tt;
            }
            if ((has & ((1u << PT_Q) | (1u << PT_P) | (1u << PT_A))) && slide_mask(P, c, c) != 0) return true;
            if ((has & (1u << PT_B)) && (climb || has_beetle(P, c))) return true;
            if ((has & (1u << PT_G)) && (jump || has_hopper(P, c))) return true;
            if ((has & (1u << PT_S)) && has_spider(P, c)) return true;
            if ((has & (1u << PT_L)) && has_ladybug(P, c)) return true;
            return false;
        }
        default: return false;
    }
}

// Can the actor at a throw the piece at t (an on-grid neighbour of a)?
// (has_pillbug_throw_for_target, move_gen.cuh:742-769)
HW_INL bool throwable(const Pos& P, int a, int dt) {
    int t = step(a, dt);
    if (!pb_get(P.occ, t) || P.hgt(t) != 1) return false;
    if (P.stun != 0xFFFF && (int)P.stun == t) return false;
    if (pb_get(P.pin, t)) return false;
    int ph = P.hgt(a);
    int back = (dt + 3) % 6;
    uint32_t gt = grid6(t);
    int lift = max(P.hgt(t) - 1, ph);
    int cwh = ((gt >> ((back + 5) % 6)) & 1u) ? P.hgt(step(t, (back + 5) % 6)) : 0;
    int ccwh = ((gt >> ((back + 1) % 6)) & 1u) ? P.hgt(step(t, (back + 1) % 6)) : 0;
    if (cwh > lift && ccwh > lift) return false;
    uint32_t ga = grid6(a);
    uint32_t oa = nbo(P, a);
    uint32_t nha = nbr_heights(P, a, ga);
    for (int dd = 0; dd < 6; dd++) {
        if (!((ga >> dd) & 1u) || dd == dt || ((oa >> dd) & 1u)) continue;
        if (!gate_high(nha, dd, ph)) return true;
    }
    return false;
}

// What the compact successor list (generate_fnn_feature_moves,
// move_gen.cuh:1416-1563) contributes to the features: its distinct
// placement cells and, per (type, owner) bucket, whether any MOVE entry
// exists (the list keeps one entry per bucket, so can_move is 0 or 1).
// Returns the bucket mask; *n_place gets the placement-cell count.
HW_INL uint32_t compact_summary(Pos& P, int lane, int* n_place) {
    *n_place = 0;
    if (P.result != 0) return 0;
    const int me = P.turn & 1;
    const int ptn = P.turn >> 1;
    const bool queen_down = (P.qplaced >> me) & 1;
    const bool queen_now = (ptn == 3) && !queen_down;
    const uint32_t held = hand_mask(P, me);
    const bool any = ((queen_now ? (held & 1u) : held) & ~(ptn == 0 ? 1u : 0u)) != 0;
    const int l = gl(lane);
    uint32_t pw = 0;
    if (any && l < 18) {
        if (P.turn == 0) {
            pw = (l == (264 >> 5)) ? (1u << (264 & 31)) : 0u;
        } else if (P.turn == 1) {
            pw = nbr_union_word(P.occ, l) & ~P.occ[l + 1];
        } else {
            const uint32_t* mine = me ? P.bt : P.wt;
            const uint32_t* theirs = me ? P.wt : P.bt;
            pw = nbr_union_word(mine, l) & ~nbr_union_word(theirs, l) & ~P.occ[l + 1];
        }
    }
    int npos = grp_sum(__popc(pw), lane);
    *n_place = npos;
    if (!queen_down || npos >= kMaxLegal) return 0;
    // one lane per occupied cell (rank l): own movable pieces and throw actors
    uint32_t bucket = 0;
    const bool occupied = l < P.n_occ;
    const int c = occupied ? P.occ_cells[l] : 0;
    const bool flat = grp_ballot(occupied && P.hgt(c) > 1, lane) == 0;  // no stack on the board
    const bool inner = grp_ballot(l < 18 && (P.occ[l + 1] & kEdgeMask.m[l]) != 0u, lane) == 0;  // none on the border
    if (occupied) {
        int tb = P.tp(c);
        int t = tb & 15;
        if (((tb >> 4) & 1) == me) {
            bool stunned = P.stun != 0xFFFF && (int)P.stun == c;
            const bool climb = P.hgt(c) == 1 && (P.sm[c] != 0 || (flat && P.nbd[l] != 0));
            const bool jump = inner && P.nbd[l] != 0;
            if (!stunned && !pb_get(P.pin, c) && piece_has_move(P, c, t, climb, jump))
                bucket |= 1u << ((t - 1) * 2 + me);
            bool actor = (t == PT_P) || (t == PT_M && P.hgt(c) == 1 && touches_top_pillbug(P, c));
            if (actor) {
                uint32_t oa = nbo(P, c);
                while (oa) {
                    int dt = __ffs(oa) - 1;
                    oa &= oa - 1;
                    if (throwable(P, c, dt)) {
                        int tb2 = P.tp(step(c, dt));
                        bucket |= 1u << (((tb2 & 15) - 1) * 2 + ((tb2 >> 4) & 1));
                    }
                }
            }
        }
    }
    return grp_or(bucket);
}

// has_queen_escape_move (move_gen.cuh:771-821); wave-uniform result
HW_INL bool queen_escape(const Pos& P, int lane) {
    const int me = P.turn & 1;
    if (!((P.qplaced >> me) & 1)) return false;
    int q = P.queen[me];
    if (q >= kCells || !pb_get(P.occ, q)) return false;
    int tq = P.tp(q);
    const int l = gl(lane);
    bool ok = false;
    if (l == 0) {
        ok = (tq & 15) == PT_Q && ((tq >> 4) & 1) == me && !pb_get(P.pin, q) && slide_mask(P, q, q) != 0;
    } else if (l < P.n_occ + 1) {
        int c = P.occ_cells[l - 1];
        int tb = P.tp(c);
        int t = tb & 15;
        if (((tb >> 4) & 1) == me && ((t == PT_P) || (t == PT_M && P.hgt(c) == 1 && touches_top_pillbug(P, c)))) {
            uint32_t bit = dir_bit_to(c, q, grid6(c));
            if (bit) ok = throwable(P, c, __ffs(bit) - 1);
        }
    }
    return grp_ballot(ok, lane) != 0;
}

// ---------------------------------------------------------------- apply
// apply_move (hive_state.cuh:497-517) on the LDS board, run by one lane.
// S is the row the LDS board was loaded from; the piece revealed when a
// stack's top leaves is read from it (levels under the top are unchanged by
// a single move).  With kResult false the surrounded-queen test that sets
// the result is left to ringed_result, run by the group once the
// occupied-neighbour masks of the new board are built.
HW_INL void pb_set(uint32_t* pb, int c) { pb[(c >> 5) + 1] |= 1u << (c & 31); }
HW_INL void pb_clr(uint32_t* pb, int c) { pb[(c >> 5) + 1] &= ~(1u << (c & 31)); }

HW_INL void set_top_colour(Pos& P, int c, int col) {
    if (col) { pb_set(P.bt, c); pb_clr(P.wt, c); }
    else { pb_set(P.wt, c); pb_clr(P.bt, c); }
}

HW_INL bool queen_ringed(const Pos& P, int col) {
    if (!((P.qplaced >> col) & 1)) return false;
    int q = P.queen[col];
    if (q >= kCells) return false;
    return __popc(nbr_bits(P.occ, q)) == 6;
}

template <bool kResult = true>
HW_INL void apply_on_board(Pos& P, const uint8_t* __restrict__ S, int type, int pt, int from, int to) {
    const int me = P.turn & 1;
    if (type == MV_PLACE) {
        if (to < kCells && pt >= PT_Q && pt <= PT_P && P.hgt(to) < 5) {
            P.set_cell(to, P.hgt(to) + 1, pt | (me << 4));
            pb_set(P.occ, to);
            set_top_colour(P, to, me);
            if (pt == PT_Q) {
                P.queen[me] = (uint16_t)to;
                P.qplaced |= (uint8_t)(1 << me);
            }
            P.hand[me][pt - 1] = (uint8_t)(P.hand[me][pt - 1] - 1);
        }
        P.stun = 0xFFFF;
    } else if (type == MV_MOVE) {
        if (from < kCells && to < kCells) {
            if (P.hgt(from) > 0 && P.hgt(from) <= 5 && P.hgt(to) < 5) {  // heights above 5 never occur
                int b = P.tp(from);
                int hf = P.hgt(from) - 1;
                if (hf == 0) {
                    P.set_cell(from, 0, 0);
                    pb_clr(P.occ, from); pb_clr(P.wt, from); pb_clr(P.bt, from);
                } else {
                    int under = S[(hf - 1) * kCells + from];
                    P.set_cell(from, hf, under);
                    set_top_colour(P, from, (under >> 4) & 1);
                }
                int ht = P.hgt(to);
                P.set_cell(to, ht + 1, b);
                pb_set(P.occ, to);
                set_top_colour(P, to, (b >> 4) & 1);
                if ((b & 15) == PT_Q) P.queen[(b >> 4) & 1] = (uint16_t)to;
            }
            P.stun = (uint16_t)to;
        }
    } else {
        P.stun = 0xFFFF;
    }
    P.turn = (uint16_t)(P.turn + 1);
    if (!kResult) return;
    bool w = queen_ringed(P, 0), k = queen_ringed(P, 1);
    if (w && k) P.result = 3;
    else if (w) P.result = 2;
    else if (k) P.result = 1;
}

// apply_on_board for a board that is also kept as a state row: the LDS board
// changes as apply_on_board changes it, and the row (global memory) receives
// the bytes that changed -- the stack byte, height and bitboard words of the
// cell the piece left and of the cell it reached, the metadata words -- so
// that it holds what RowView::apply leaves (states of init/apply: stack bytes
// fit the board's five top bits, heights stay below 8).  The board is read
// from LDS; the row is read only for the piece revealed under a leaving top.
// Run by one lane.
HW_INL void apply_mirrored(Pos& P, uint8_t* __restrict__ row, int type, int pt, int from, int to) {
    const int hf0 = from < kCells ? P.hgt(from) : 0;
    const int ht0 = to < kCells ? P.hgt(to) : 0;
    apply_on_board<true>(P, row, type, pt, from, to);
    uint32_t* meta = reinterpret_cast<uint32_t*>(row + OFF_QUEEN);  // queens, hands, turn / flags
    const uint32_t* hand32 = reinterpret_cast<const uint32_t*>(P.hand);
    meta[0] = (uint32_t)P.queen[0] | ((uint32_t)P.queen[1] << 16);
    meta[1] = hand32[0];
    meta[2] = hand32[1];
    meta[3] = hand32[2];
    meta[4] = hand32[3];
    meta[5] = (uint32_t)P.turn | ((uint32_t)P.qplaced << 16) | ((uint32_t)P.result << 24);
    *reinterpret_cast<uint16_t*>(row + OFF_STUN) = P.stun;
    auto words = [&](int c) {
        const int w = c >> 5;
        reinterpret_cast<uint32_t*>(row + OFF_OCC)[w] = P.occ[w + 1];
        reinterpret_cast<uint32_t*>(row + OFF_WTOP)[w] = P.wt[w + 1];
        reinterpret_cast<uint32_t*>(row + OFF_BTOP)[w] = P.bt[w + 1];
    };
    if (type == MV_MOVE && from < kCells && P.hgt(from) != hf0) {  // the piece left: hf0 - 1 high now
        row[(hf0 - 1) * kCells + from] = 0;
        row[OFF_HEIGHT + from] = (uint8_t)(hf0 - 1);
        words(from);
    }
    if (to < kCells && P.hgt(to) != ht0) {  // a piece arrived: ht0 + 1 high now
        row[ht0 * kCells + to] = (uint8_t)P.tp(to);
        row[OFF_HEIGHT + to] = (uint8_t)(ht0 + 1);
        words(to);
    }
}

// The result apply_on_board<true> sets, from the masks build_cell_masks left:
// a placed queen is surrounded when the occupied-neighbour mask of its cell
// has all six on-grid directions (queen_ringed's test; off-grid directions
// are never set).  Every occupied cell is ranked: a board of init/apply
// holds at most 28 pieces, and a placed queen's cell stays occupied.  Lane 0
// writes the result before the next barrier.
HW_INL void ringed_result(Pos& P, int lane) {
    const int l = gl(lane);
    bool w = false, k = false;
    if (l < P.n_occ && P.nbd[l] == 63u) {
        const int c = P.occ_cells[l];
        w = (P.qplaced & 1) && c == (int)P.queen[0];
        k = (P.qplaced & 2) && c == (int)P.queen[1];
    }
    const bool W = grp_ballot(w, lane) != 0, K = grp_ballot(k, lane) != 0;
    if (gl(lane) == 0 && (W || K)) P.result = (uint8_t)(W && K ? 3 : W ? 2 : 1);
}

// ---------------------------------------------------------------- programs
// Whole-position programs run by all 64 lanes of a wave; the kernels in
// hive_engine.hip are thin launch wrappers around them.

// board prepared for move generation (load_position done, moves applied)
HW_INL void prepare_loaded(Pos& P, int lane) {
    build_occ_list(P, lane);
    __syncthreads();
    build_cell_masks(P, lane);
    articulation(P, lane);
    __syncthreads();
}

HW_INL void prepare(Pos& P, const uint8_t* __restrict__ S, int lane) {
    load_position(P, S, lane);
    __syncthreads();
    prepare_loaded(P, lane);
}

// run_legal on a board already loaded (load_position or moves applied since,
// behind a barrier); S is the state row it stands for (stacked levels).
template <bool WithMoves, bool WithFeat, bool WithAct>
HW_INL void run_legal_loaded(Pos& P, const uint8_t* __restrict__ S, int lane, uint8_t* __restrict__ moves_row,
                             int32_t* __restrict__ n_slot, float* __restrict__ feat_row,
                             int32_t* __restrict__ act_row, bool pad = true) {
    prepare_loaded(P, lane);
    ListInfo L = generate_legal(P, lane);
    place_list(P, lane);
    if (WithFeat) sources_clear(P, lane);
    int cq = 0, cr = 0;
    if (WithAct) {
        centroid(P, lane, cq, cr);
        if (gl(lane) < L.n_pieces) P.piece_win[gl(lane)] = (int16_t)window17(P.piece_cell[gl(lane)], cq, cr);
    }
    __syncthreads();
    if (moves_row) emit_list<WithMoves, WithAct, WithFeat>(P, L, lane, moves_row, act_row, cq, cr, pad);
    if (gl(lane) == 0 && n_slot) *n_slot = L.n;
    if (WithFeat) {
        __syncthreads();
        counters_clear(P, lane);
        __syncthreads();
        int m = L.total > 0 ? min(L.n, L.n_place) : 0;
        features_finish(P, S, feat_row, lane, kFeatGen, 0u, L.ntypes ? (m + L.ntypes - 1) / L.ntypes : 0);
    }
}

template <bool WithMoves, bool WithFeat, bool WithAct>
HW_INL void run_legal(Pos& P, const uint8_t* __restrict__ S, int lane, uint8_t* __restrict__ moves_row,
                      int32_t* __restrict__ n_slot, float* __restrict__ feat_row, int32_t* __restrict__ act_row) {
    load_position(P, S, lane);
    __syncthreads();
    run_legal_loaded<WithMoves, WithFeat, WithAct>(P, S, lane, moves_row, n_slot, feat_row, act_row);
}

HW_INL void run_extract(Pos& P, ListSets& X, const uint8_t* __restrict__ S, const uint8_t* __restrict__ M, int nl,
                        int lane, float* __restrict__ feat_row) {
    int n = nl < 0 ? 0 : (nl > kMaxLegal ? kMaxLegal : nl);
    prepare(P, S, lane);
    sources_clear(P, lane, &X);
    counters_clear(P, lane);
    __syncthreads();
    list_sources(P, M, n, lane, X);
    __syncthreads();
    features_finish(P, S, feat_row, lane, kFeatList, 0u, 0, &X);
}

// fnn_successor_features_kernel (game_logic.cu:182-229) for one (root, move),
// the root's row S already on the board
HW_INL void successor_on_board(Pos& P, const uint8_t* __restrict__ S, const uint8_t* __restrict__ m, int lane,
                               float* __restrict__ feat_row) {
    if (gl(lane) == 0) apply_on_board<false>(P, S, m[0], m[1], m[2] | (m[3] << 8), m[4] | (m[5] << 8));
    __syncthreads();
    build_occ_list(P, lane);
    __syncthreads();
    build_cell_masks(P, lane);
    ringed_result(P, lane);
    articulation(P, lane);
    __syncthreads();
    int n_place = 0;
    uint32_t bucket = compact_summary(P, lane, &n_place);
    sources_clear(P, lane);
    counters_clear(P, lane);
    __syncthreads();
    // stacked levels under a top piece are read from the root row: a single
    // move leaves every level under a top unchanged
    features_finish(P, S, feat_row, lane, kFeatBucket, bucket, n_place);
}

HW_INL void run_successor(Pos& P, const uint8_t* __restrict__ S, const uint8_t* __restrict__ m, int lane,
                          float* __restrict__ feat_row) {
    load_position(P, S, lane);
    __syncthreads();
    successor_on_board(P, S, m, lane, feat_row);
}

// Successor features of a stream of rows taken by one lane group: rows come
// in (root, slot) order, so consecutive rows mostly share their root; the
// root's row is loaded when the root changes and otherwise the board is
// restored from registers (BaseRegs).  A row at or past N produces nothing;
// a row whose root or slot is out of range gets zero features.  zero_row: a
// state row and move of zero bytes.
struct SuccessorStream {
    BaseRegs R;
    int64_t cur = -2;  // root whose base R holds (-1: the zero row)
};

// Ix: the index type of the rows and roots.  int64_t takes any batch;
// uint32_t (`narrow`, for batches whose state, move and feature offsets all
// stay below 2^32 -- the caller's check) does the row's index arithmetic in
// 32 bits.  The range checks are made on the loaded 64-bit values either way.
template <typename Ix = int64_t>
HW_INL void successor_row(Pos& P, SuccessorStream& st, const uint8_t* __restrict__ states,
                          const uint8_t* __restrict__ legal, const int64_t* __restrict__ a2r,
                          const int64_t* __restrict__ midx, Ix i, Ix N, int64_t num_roots,
                          const uint8_t* __restrict__ zero_row, int lane, float* __restrict__ feat_out) {
    const bool live = i < N;
    const int64_t r64 = live ? a2r[i] : -1;
    const int64_t m64 = live ? midx[i] : -1;
    const bool valid = (uint64_t)r64 < (uint64_t)num_roots && (uint64_t)m64 < (uint64_t)kMaxLegal;
    const Ix root = (Ix)r64, mi = (Ix)m64;
    const uint8_t* S = valid ? states + (Ix)(root * (Ix)kStateBytes) : zero_row;
    const uint8_t* m = valid ? legal + (Ix)((root * (Ix)kMaxLegal + mi) * (Ix)6) : zero_row;
    const int64_t key = valid ? r64 : -1;
    const bool fresh = key != st.cur;
    if (fresh) load_position(P, S, lane);
    else restore_base(P, st.R, lane);
    __syncthreads();
    if (fresh) save_base(P, st.R, lane);
    st.cur = key;
    __syncthreads();
    float* out = feat_out + (Ix)(i * (Ix)kFeat);
    successor_on_board(P, S, m, lane, live && valid ? out : nullptr);
    if (live && !valid)
        for (int k = gl(lane); k < kFeat; k += kW) out[k] = 0.0f;
    __syncthreads();
}

HW_INL bool run_queen_escape(Pos& P, const uint8_t* __restrict__ S, int lane) {
    prepare(P, S, lane);
    return queen_escape(P, lane);
}
// ---------------------------------------------------------------- rows
// Byte-level apply_move (hive_state.cuh:326-517) on a state row in global
// memory or LDS, run by one lane.
struct RowView {
    uint8_t* s;
    __device__ uint8_t& stack(int lv, int c) { return s[lv * kCells + c]; }
    __device__ uint8_t& h(int c) { return s[OFF_HEIGHT + c]; }
    __device__ uint64_t* bb(int off) { return reinterpret_cast<uint64_t*>(s + off); }
    __device__ void set(int off, int c) { bb(off)[c >> 6] |= 1ull << (c & 63); }
    __device__ void clr(int off, int c) { bb(off)[c >> 6] &= ~(1ull << (c & 63)); }
    __device__ bool get(int off, int c) { return (bb(off)[c >> 6] >> (c & 63)) & 1ull; }
    __device__ uint16_t& u16(int off) { return *reinterpret_cast<uint16_t*>(s + off); }
    __device__ void top_colour(int c, int col) {
        if (col) { set(OFF_BTOP, c); clr(OFF_WTOP, c); }
        else { set(OFF_WTOP, c); clr(OFF_BTOP, c); }
    }
    // occupancy word w (cells 32w .. 32w + 31) for w >= -1: word -1 is the
    // four row bytes before the bitboard (heights), whose bits only ever land
    // on off-grid directions and are masked off
    __device__ uint32_t occ_word(int w) { return *reinterpret_cast<const uint32_t*>(s + OFF_OCC + 4 * w); }
    // the queen's six on-grid neighbours all occupied, from one 64-bit window
    // of the occupancy starting at cell q - 23 (three independent word reads)
    __device__ bool ringed(int col) {
        if (!((s[OFF_QPLACED] >> col) & 1)) return false;
        int q = u16(OFF_QUEEN + 2 * col);
        if (q >= kCells) return false;
        const int lo = q - 23, w = lo >> 5, sh = lo & 31;
        uint64_t win = ((uint64_t)occ_word(w) | ((uint64_t)occ_word(w + 1) << 32)) >> sh;
        if (sh) win |= (uint64_t)occ_word(w + 2) << (64 - sh);
        return (ring_bits(win) & grid6(q)) == 63u;
    }
    __device__ void apply(int type, int pt, int from, int to) {
        int me = u16(OFF_TURN) & 1;
        if (type == MV_PLACE) {
            if (to < kCells && pt >= PT_Q && pt <= PT_P && h(to) < 5) {
                int hh = h(to);
                stack(hh, to) = (uint8_t)(pt | (me << 4));
                h(to) = (uint8_t)(hh + 1);
                if (hh == 0) set(OFF_OCC, to);
                top_colour(to, me);
                if (pt == PT_Q) {
                    u16(OFF_QUEEN + 2 * me) = (uint16_t)to;
                    s[OFF_QPLACED] |= (uint8_t)(1 << me);
                }
                s[OFF_HANDS + me * 8 + pt - 1] -= 1;
            }
            u16(OFF_STUN) = 0xFFFF;
        } else if (type == MV_MOVE) {
            if (from < kCells && to < kCells) {
                if (h(from) > 0 && h(from) <= 5 && h(to) < 5) {  // heights above 5 never occur
                    int hf = h(from);
                    uint8_t b = stack(hf - 1, from);
                    stack(hf - 1, from) = 0;
                    h(from) = (uint8_t)(hf - 1);
                    if (hf == 1) {
                        clr(OFF_OCC, from); clr(OFF_WTOP, from); clr(OFF_BTOP, from);
                    } else {
                        top_colour(from, (stack(hf - 2, from) >> 4) & 1);
                    }
                    int ht = h(to);
                    stack(ht, to) = b;
                    h(to) = (uint8_t)(ht + 1);
                    if (ht == 0) set(OFF_OCC, to);
                    top_colour(to, (b >> 4) & 1);
                    if ((b & 15) == PT_Q) u16(OFF_QUEEN + 2 * ((b >> 4) & 1)) = (uint16_t)to;
                }
                u16(OFF_STUN) = (uint16_t)to;
            }
        } else {
            u16(OFF_STUN) = 0xFFFF;
        }
        u16(OFF_TURN) = (uint16_t)(u16(OFF_TURN) + 1);
        bool w = ringed(0), k = ringed(1);
        if (w && k) s[OFF_RESULT] = 3;
        else if (w) s[OFF_RESULT] = 2;
        else if (k) s[OFF_RESULT] = 1;
    }
};

}  // namespace hw
