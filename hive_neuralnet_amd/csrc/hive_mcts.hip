// hive_mcts.hip -- MCTS tree kernels over the reference's structure-of-arrays
// tree (mcts_tree.cuh:31-45): select with root slots / root mask, replay,
// dense-prior expansion, fused expansion + backup, root noise.
//
// Order of effect.  The reference runs one thread per simulation with
// atomics, so simulations of one game race on virtual-loss reads, on which
// of them expands a shared leaf, on node-id allocation and on float
// summation order (mcts_tree.cuh:773-786,1001-1020,1166-1186).  Here one
// wavefront owns one game and applies that game's simulations in
// simulation-index order (sim = k*B + game, k = 0, 1, ...): each selection
// sees the virtual losses of earlier ones, the earliest simulation reaching
// an unexpanded leaf expands it, node ids are handed out in that order and
// every float update of a node happens in that order.  Within one
// simulation the lanes split the per-child work (PUCT over a node's
// children, initialising a new node's children).  With one simulation per
// root candidate per call the result equals every interleaving of the
// reference up to node numbering.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hive_gpu.h"
#include "hive_leaf.hpp"
#include "hive_phases.hpp"

using namespace hw;

namespace {

constexpr int kDepth = 128;  // MAX_TREE_DEPTH (mcts_tree.cuh:27)

struct Tree {
    int32_t* vc;
    float* tv;
    float* pr;
    int32_t* pa;
    float* vq;
    uint8_t* mb;
    int32_t* ai;
    int32_t* fc;
    int32_t* nc;
    int8_t* it;
    float* tval;
    int32_t* cnt;
    float* ciq;
    int64_t M;
};

Tree to_tree(const hg_tree* t) {
    return Tree{t->visit_count, t->total_value, t->prior, t->parent_idx, t->virtual_q_penalty, t->move_bytes,
                t->action_idx, t->first_child, t->num_children, t->is_terminal, t->terminal_value,
                t->node_count, t->child_init_q, t->max_nodes};
}

// puct_score (mcts_tree.cuh:55-67), evaluated in the same operation order
__device__ __forceinline__ float puct(const Tree& T, int64_t pi, int64_t ci, float c_puct) {
    int n = T.vc[ci];
    float q = n > 0 ? (-T.tv[ci] / (float)n) : 0.0f;
    q -= T.vq[ci];
    float explore = c_puct * T.pr[ci] * sqrtf((float)T.vc[pi]) / (1.0f + (float)n);
    return q + explore;
}

// first maximum of score over the lanes' candidates (score must beat -1e30)
__device__ __forceinline__ int wave_argmax_first(float score, int idx) {
    bool ok = score > -1e30f;  // NaN and the -1e30 floor never win (strict '>' from -1e30)
    float s = ok ? score : -INFINITY;
    int i = ok ? idx : 0x7fffffff;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float s2 = __shfl_xor(s, o, 64);
        int i2 = __shfl_xor(i, o, 64);
        if (s2 > s || (s2 == s && i2 < i)) { s = s2; i = i2; }
    }
    return i == 0x7fffffff ? -1 : i;
}

// deterministic_completed_q_child (mcts_tree.cuh:77-143), one lane, child order
HW_INL int completed_q_child(const Tree& T, int64_t g0, int first, int count, float sigma) {
    float sum_visits = 0.0f;
    for (int c = 0; c < count; c++) {
        if (first + c < 0 || first + c >= T.M) break;
        sum_visits += (float)T.vc[g0 + first + c];
    }
    float mx = -1e30f;
    for (int c = 0; c < count; c++) {
        if (first + c < 0 || first + c >= T.M) break;
        int64_t ci = g0 + first + c;
        float visits = (float)T.vc[ci];
        float q = visits > 0.0f ? (-T.tv[ci] / visits) : T.ciq[ci];
        q -= T.vq[ci];
        float lq = logf(fmaxf(T.pr[ci], 1e-20f)) + sigma * q;
        if (lq > mx) mx = lq;
    }
    float se = 0.0f;
    for (int c = 0; c < count; c++) {
        if (first + c < 0 || first + c >= T.M) break;
        int64_t ci = g0 + first + c;
        float visits = (float)T.vc[ci];
        float q = visits > 0.0f ? (-T.tv[ci] / visits) : T.ciq[ci];
        q -= T.vq[ci];
        se += expf(logf(fmaxf(T.pr[ci], 1e-20f)) + sigma * q - mx);
    }
    se = fmaxf(se, 1e-20f);
    int best = -1;
    float bs = -1e30f;
    float denom = 1.0f + sum_visits;
    for (int c = 0; c < count; c++) {
        if (first + c < 0 || first + c >= T.M) break;
        int64_t ci = g0 + first + c;
        float visits = (float)T.vc[ci];
        float q = visits > 0.0f ? (-T.tv[ci] / visits) : T.ciq[ci];
        q -= T.vq[ci];
        float pi0 = expf(logf(fmaxf(T.pr[ci], 1e-20f)) + sigma * q - mx) / se;
        float score = pi0 - (visits / denom);
        if (score > bs) { bs = score; best = first + c; }
    }
    return best;
}

struct SelectOut {
    int32_t* leaf;
    uint8_t* paths;
    int32_t* plen;
    int32_t* vl;
    int32_t* vlen;
    int tails = 1;  // 0: the rows past the recorded entries are left as they are
};

// Zeros past the recorded entries of a simulation's path rows (move bytes
// from plen, node ids from vlen), so the dense selects write whole rows and
// their callers need not clear the outputs.  The simulation wave, whose
// readers stop at the lengths, leaves the tails (O.tails = 0).
__device__ __forceinline__ void zero_tails(const SelectOut& O, int64_t sim, int plen, int vlen, int lane) {
    if (!O.tails) return;
    uint16_t* pw = reinterpret_cast<uint16_t*>(O.paths + sim * kDepth * 6);
    for (int k = 3 * plen + lane; k < 3 * kDepth; k += 64) pw[k] = 0;
    int32_t* vw = O.vl + sim * kDepth;
    for (int k = vlen + lane; k < kDepth; k += 64) vw[k] = 0;
}

__device__ __forceinline__ void empty_sim(const SelectOut& O, int64_t sim, int lane) {
    if (lane == 0) {
        O.leaf[sim] = -1;
        O.plen[sim] = 0;
        O.vlen[sim] = 0;
    }
}

// an empty simulation of a dense select: whole rows
__device__ __forceinline__ void empty_sim_rows(const SelectOut& O, int64_t sim, int lane) {
    empty_sim(O, sim, lane);
    zero_tails(O, sim, 0, 0, lane);
}

// Enter `node` below the root (virtual loss or q penalty, path records).
__device__ __forceinline__ void enter(const Tree& T, int64_t g0, int node, bool det, float q_penalty,
                                      const SelectOut& O, int64_t sim, int& plen, int& vlen, int lane) {
    if (lane == 0) {
        int64_t ni = g0 + node;
        if (det) {
            T.vc[ni] += 1;
            T.vq[ni] += q_penalty;
        } else {
            T.vc[ni] += 1;
            T.tv[ni] += -1.0f;
        }
        if (vlen < kDepth) O.vl[sim * kDepth + vlen] = node;
        if (plen < kDepth) {
            const uint8_t* src = T.mb + ni * 6;
            uint8_t* dst = O.paths + (sim * kDepth + plen) * 6;
            for (int b = 0; b < 6; b++) dst[b] = src[b];
        }
    }
    vlen = vlen < kDepth ? vlen + 1 : vlen;
    plen = plen < kDepth ? plen + 1 : plen;
    __syncthreads();  // later reads of this game's statistics see the update
}

// What the descent reads of a child, loaded in one round trip by the lane
// that scores it: statistics for PUCT and the virtual loss, the child's own
// children (the next level) and its move bytes (the path record).
struct ChildRec {
    int vc;
    float tv, vq, pr;
    int fc, nc;
    int it;
    uint16_t mb0, mb1, mb2;
};

__device__ __forceinline__ ChildRec load_rec(const Tree& T, int64_t ci) {
    ChildRec r;
    r.vc = T.vc[ci];
    r.tv = T.tv[ci];
    r.vq = T.vq[ci];
    r.pr = T.pr[ci];
    r.fc = T.fc[ci];
    r.nc = T.nc[ci];
    r.it = T.it[ci];
    const uint16_t* m = reinterpret_cast<const uint16_t*>(T.mb + ci * 6);
    r.mb0 = m[0];
    r.mb1 = m[1];
    r.mb2 = m[2];
    return r;
}

__device__ __forceinline__ ChildRec shfl_rec(const ChildRec& r, int src) {
    ChildRec o;
    o.vc = __shfl(r.vc, src, 64);
    o.tv = __shfl(r.tv, src, 64);
    o.vq = __shfl(r.vq, src, 64);
    o.pr = __shfl(r.pr, src, 64);
    o.fc = __shfl(r.fc, src, 64);
    o.nc = __shfl(r.nc, src, 64);
    o.it = __shfl(r.it, src, 64);
    o.mb0 = (uint16_t)__shfl((int)r.mb0, src, 64);
    o.mb1 = (uint16_t)__shfl((int)r.mb1, src, 64);
    o.mb2 = (uint16_t)__shfl((int)r.mb2, src, 64);
    return o;
}

// puct_score (mcts_tree.cuh:55-67) of a loaded child, parent visits pvc
__device__ __forceinline__ float puct_rec(const ChildRec& r, int pvc, float c_puct) {
    int n = r.vc;
    float q = n > 0 ? (-r.tv / (float)n) : 0.0f;
    q -= r.vq;
    float explore = c_puct * r.pr * sqrtf((float)pvc) / (1.0f + (float)n);
    return q + explore;
}

// Enter `node` (record r, as loaded) below the root: virtual loss or q
// penalty written from the loaded values (no other wave touches this node
// during the kernel, and this simulation reads it again only as the parent,
// whose visit count the caller carries in a register), path records.
__device__ __forceinline__ void enter_rec(const Tree& T, int64_t g0, int node, const ChildRec& r, bool det,
                                          float q_penalty, const SelectOut& O, int64_t sim, int& plen, int& vlen,
                                          int lane) {
    if (lane == 0) {
        int64_t ni = g0 + node;
        T.vc[ni] = r.vc + 1;
        if (det) T.vq[ni] = r.vq + q_penalty;
        else T.tv[ni] = r.tv + -1.0f;
        if (vlen < kDepth) O.vl[sim * kDepth + vlen] = node;
        if (plen < kDepth) {
            uint16_t* dst = reinterpret_cast<uint16_t*>(O.paths + (sim * kDepth + plen) * 6);
            dst[0] = r.mb0;
            dst[1] = r.mb1;
            dst[2] = r.mb2;
        }
    }
    vlen = vlen < kDepth ? vlen + 1 : vlen;
    plen = plen < kDepth ? plen + 1 : plen;
}

// PUCT descent below `node` (mcts_tree.cuh:895-950 / 729-795 below the root):
// r is the record of `node`, pvc its visit count as this simulation left it.
// One round trip of loads per level: each lane loads its children's records,
// the winner's record is broadcast and carries the next level.
HW_INL int descend_rec(const Tree& T, int64_t g0, int node, ChildRec r, int pvc, int first_iter, float c_puct,
                       bool det, float sigma, float q_penalty, const SelectOut& O, int64_t sim, int& plen, int& vlen,
                       int lane) {
    for (int it = first_iter; it < kDepth; it++) {
        const int cfc = r.fc, cnc = r.nc;
        if (cfc < 0 || r.it || cnc == 0) break;
        if (cnc <= 0 || cnc > 1024) break;
        int best;
        ChildRec win;
        if (det) {
            int b = 0;
            if (lane == 0) b = completed_q_child(T, g0, cfc, cnc, sigma);
            best = __shfl(b, 0, 64);
            if (best < 0) break;
            win = load_rec(T, g0 + best);
        } else {
            float bs = -INFINITY;
            int bi = 0x7fffffff;
            ChildRec mine = r;
            for (int c = lane; c < cnc; c += 64) {
                int child = cfc + c;
                if (child < 0 || child >= T.M) break;
                ChildRec cr = load_rec(T, g0 + child);
                float sc = puct_rec(cr, pvc, c_puct);
                if (sc > -1e30f && (sc > bs || (sc == bs && c < bi))) {
                    bs = sc;
                    bi = c;
                    mine = cr;
                }
            }
            int c = wave_argmax_first(bs, bi);
            if (c < 0) break;
            best = cfc + c;
            win = shfl_rec(mine, c & 63);
        }
        node = best;
        enter_rec(T, g0, node, win, det, q_penalty, O, sim, plen, vlen, lane);
        pvc = win.vc + 1;
        r = win;
    }
    return node;
}


// The simulations of one (game, candidate) wave in PUCT mode with the
// candidate's root child and that child's children held in registers for the
// whole wave: every simulation enters the same root child and scores the same
// children, so their records are loaded once, scored and updated in
// registers (the same float operations in the same order as through memory:
// no other wave touches this subtree during the kernel), and written back
// once after the wave's last simulation.  Levels below go through memory as
// before.  Children: up to kKidRegs per lane (64 kKidRegs in all).
constexpr int kKidRegs = 4;
// a child record in eight registers (terminal flag and move bytes packed)
struct KidRec {
    int vc;
    float tv, vq, pr;
    int fc, nc;
    uint32_t mb01, mb2it;
};
__device__ __forceinline__ KidRec pack_kid(const ChildRec& r) {
    return KidRec{r.vc, r.tv, r.vq, r.pr, r.fc, r.nc, (uint32_t)r.mb0 | ((uint32_t)r.mb1 << 16),
                  (uint32_t)r.mb2 | ((uint32_t)(r.it != 0) << 16)};
}
__device__ __forceinline__ ChildRec unpack_kid(const KidRec& k) {
    ChildRec r;
    r.vc = k.vc;
    r.tv = k.tv;
    r.vq = k.vq;
    r.pr = k.pr;
    r.fc = k.fc;
    r.nc = k.nc;
    r.it = (int)(k.mb2it >> 16);
    r.mb0 = (uint16_t)k.mb01;
    r.mb1 = (uint16_t)(k.mb01 >> 16);
    r.mb2 = (uint16_t)k.mb2it;
    return r;
}
__device__ __forceinline__ float puct_kid(const KidRec& r, int pvc, float c_puct) {
    int n = r.vc;
    float q = n > 0 ? (-r.tv / (float)n) : 0.0f;
    q -= r.vq;
    float explore = c_puct * r.pr * sqrtf((float)pvc) / (1.0f + (float)n);
    return q + explore;
}
__device__ __forceinline__ KidRec shfl_kid(const KidRec& r, int src) {
    return KidRec{__shfl(r.vc, src, 64), __shfl(r.tv, src, 64), __shfl(r.vq, src, 64), __shfl(r.pr, src, 64),
                  __shfl(r.fc, src, 64), __shfl(r.nc, src, 64), (uint32_t)__shfl((int)r.mb01, src, 64),
                  (uint32_t)__shfl((int)r.mb2it, src, 64)};
}
// Level 3 of a simulation in select_slot_cached: the children of the level-2
// node (k2-th child of the root child, record `win` as the simulation found
// it) scored from an LDS copy when they are at most 64 and all inside the
// pool.  The copies of the level-2 nodes the wave's simulations pass through
// are kept in kC3 entries (tag = k2, replaced in turn), loaded on the first
// visit and updated with the virtual loss as memory is (written through), so
// a later simulation through the same node scores the same records without
// a memory round trip.  No other wave touches this subtree during the
// kernel, and the tree's structure does not change in it.  Then the descent
// goes on through memory (descend_rec) from level 4.
constexpr int kC3 = 4;
HW_INL int descend_level3(const Tree& T, int64_t g0, int node2, int k2, const ChildRec& win, float c_puct,
                          const SelectOut& O, int64_t sim, int& plen, int& vlen, int lane, KidRec (*c3)[64],
                          int* tag3, int& next3) {
    const int cfc = win.fc, cnc = win.nc;
    const bool cacheable = !(cfc < 0 || win.it || cnc == 0) && cnc <= 64 && (int64_t)cfc + cnc <= T.M;
    // where the descent through memory starts: level 3 below node2, or level 4
    // below the cached level's winner (first_iter kDepth: no descent at all)
    int node = node2, first = 2;
    ChildRec r = win;
    if (cacheable) {
        int e = -1;
#pragma unroll
        for (int i = 0; i < kC3; i++)
            if (tag3[i] == k2) e = i;
        if (e < 0) {  // first visit: the children's records as memory holds them now
            e = next3;
            next3 = next3 == kC3 - 1 ? 0 : next3 + 1;
            tag3[e] = k2;
            if (lane < cnc) c3[e][lane] = pack_kid(load_rec(T, g0 + cfc + lane));
        }
        KidRec mine = c3[e][lane];
        float bs = -INFINITY;
        int bi = 0x7fffffff;
        if (lane < cnc) {
            const float sc = puct_kid(mine, win.vc + 1, c_puct);
            if (sc > -1e30f) {
                bs = sc;
                bi = lane;
            }
        }
        const int k3 = wave_argmax_first(bs, bi);
        first = kDepth;
        if (k3 >= 0) {
            r = unpack_kid(shfl_kid(mine, k3));
            node = cfc + k3;
            if (lane == k3) {  // the copy takes the virtual loss enter_rec writes to memory
                mine.vc = r.vc + 1;
                mine.tv = r.tv + -1.0f;
                c3[e][lane] = mine;
            }
            enter_rec(T, g0, node, r, false, 0.0f, O, sim, plen, vlen, lane);
            first = 3;
        }
    }
    return descend_rec(T, g0, node, r, r.vc + 1, first, c_puct, false, 0.0f, 0.0f, O, sim, plen, vlen, lane);
}

HW_INL void select_slot_cached(const Tree& T, int64_t g0, int node1, ChildRec r1, int64_t g, int64_t B, int c,
                               int C, int64_t rounds, float c_puct, const SelectOut& O, int lane) {
    __shared__ KidRec c3[kC3][64];
    int tag3[kC3];
#pragma unroll
    for (int i = 0; i < kC3; i++) tag3[i] = -1;
    int next3 = 0;
    const int fc1 = r1.fc, nc1 = r1.nc;
    const bool grown = !(fc1 < 0 || r1.it || nc1 == 0) && !(nc1 <= 0 || nc1 > 1024);
    // the children that descend_rec would score: stop at the first one outside the pool
    int nk = 0;
    if (grown) nk = (int64_t)fc1 + nc1 <= T.M ? nc1 : (fc1 < T.M ? (int)(T.M - fc1) : 0);
    KidRec kid[kKidRegs];
    uint32_t dirty = 0;
#pragma unroll
    for (int j = 0; j < kKidRegs; j++) {
        const int k = lane + 64 * j;
        kid[j] = pack_kid(k < nk ? load_rec(T, g0 + fc1 + k) : r1);
    }
    for (int64_t kk = c; kk < rounds; kk += C) {
        const int64_t sim = kk * B + g;
        int plen = 0, vlen = 0;
        // level 1: the root child (virtual loss in registers, path records in memory)
        if (lane == 0) {
            O.vl[sim * kDepth] = node1;
            uint16_t* dst = reinterpret_cast<uint16_t*>(O.paths + sim * kDepth * 6);
            dst[0] = r1.mb0;
            dst[1] = r1.mb1;
            dst[2] = r1.mb2;
        }
        plen = vlen = 1;
        const int pvc = r1.vc + 1;
        r1.vc = pvc;
        r1.tv = r1.tv + -1.0f;
        int node = node1;
        if (grown && nk > 0) {
            // level 2: PUCT over the children in registers, first maximum
            float bs = -INFINITY;
            int bi = 0x7fffffff;
            int bj = 0;
#pragma unroll
            for (int j = 0; j < kKidRegs; j++) {
                const int k = lane + 64 * j;
                if (k < nk) {
                    const float sc = puct_kid(kid[j], pvc, c_puct);
                    if (sc > -1e30f && (sc > bs || (sc == bs && k < bi))) {
                        bs = sc;
                        bi = k;
                        bj = j;
                    }
                }
            }
            const int k2 = wave_argmax_first(bs, bi);
            if (k2 >= 0) {
                KidRec mine = kid[0];
#pragma unroll
                for (int j = 1; j < kKidRegs; j++)
                    if (bj == j) mine = kid[j];
                const ChildRec win = unpack_kid(shfl_kid(mine, k2 & 63));
                node = fc1 + k2;
                if (lane == (k2 & 63)) {
#pragma unroll
                    for (int j = 0; j < kKidRegs; j++)
                        if (j == (k2 >> 6)) {
                            kid[j].vc = win.vc + 1;
                            kid[j].tv = win.tv + -1.0f;
                            dirty |= 1u << j;
                        }
                }
                if (lane == 0) {
                    O.vl[sim * kDepth + 1] = node;
                    uint16_t* dst = reinterpret_cast<uint16_t*>(O.paths + (sim * kDepth + 1) * 6);
                    dst[0] = win.mb0;
                    dst[1] = win.mb1;
                    dst[2] = win.mb2;
                }
                plen = vlen = 2;
                node = descend_level3(T, g0, node, k2, win, c_puct, O, sim, plen, vlen, lane, c3, tag3, next3);
            }
        }
        __syncthreads();  // the next simulation reads this one's statistics below level 2
        if (lane == 0) {
            O.leaf[sim] = node;
            O.plen[sim] = plen;
            O.vlen[sim] = vlen;
        }
        zero_tails(O, sim, plen, vlen, lane);
    }
    // write back the statistics held in registers
    if (lane == 0) {
        T.vc[g0 + node1] = r1.vc;
        T.tv[g0 + node1] = r1.tv;
    }
#pragma unroll
    for (int j = 0; j < kKidRegs; j++)
        if ((dirty >> j) & 1u) {
            const int64_t ci = g0 + fc1 + lane + 64 * j;
            T.vc[ci] = kid[j].vc;
            T.tv[ci] = kid[j].tv;
        }
}

// mcts_select_with_root_slots_kernel (mcts_tree.cuh:811-955), one wave per
// (game, candidate).  A simulation forced into root child fc + slot touches
// only that child's subtree (the root itself is not entered), so the
// candidates of a game with distinct slots are independent: wave (g, c)
// runs candidate c's simulations sim = (w*C + c)*B + g in order of w, which
// is the game's simulation order restricted to them.  A game whose slot list
// repeats a slot runs all its simulations in one wave, in order.
__global__ __launch_bounds__(64) void k_select_slots(Tree T, const int8_t* __restrict__ game_active,
                                                     const int32_t* __restrict__ root_nodes,
                                                     const int32_t* __restrict__ root_slots, int C, int max_root,
                                                     float c_puct, int64_t B, int64_t total, int det, float sigma,
                                                     float q_penalty, SelectOut O) {
    const int64_t g = blockIdx.x / C;
    const int c = (int)(blockIdx.x % C);
    const int lane = threadIdx.x;
    if (g >= B) return;
    const int lane_slot = lane < C ? root_slots[g * C + lane] : -1;
    bool dup = false;
    if (C <= 64) {  // the slots are in lanes: compare them by shuffles
        for (int c2 = 1; c2 < C; c2++) {
            const int s2 = __shfl(lane_slot, c2, 64);
            dup |= lane < c2 && lane_slot >= 0 && lane_slot == s2;
        }
    } else {
        for (int c1 = lane; c1 < C; c1 += 64) {
            int s1 = root_slots[g * C + c1];
            if (s1 < 0) continue;
            for (int c2 = c1 + 1; c2 < C; c2++) dup |= root_slots[g * C + c2] == s1;
        }
    }
    dup = __ballot(dup) != 0;
    if (dup && c != 0) return;
    const int64_t g0 = g * T.M;
    const int64_t rounds = total / B;  // simulations per game
    // the game's root and slots do not change during the kernel
    const bool active = game_active[g] != 0;
    const int root = root_nodes[g];
    const int64_t ri = g0 + root;
    const int rfc = T.fc[ri], rnc = T.nc[ri];
    const bool rterm = T.it[ri] != 0;
    if (!det && !dup && active) {  // one root child for the whole wave: its level in registers
        const int slot = C <= 64 ? __shfl(lane_slot, c, 64) : root_slots[g * C + c];
        const int node1 = rfc + slot;
        if (slot >= 0 && slot < max_root && !(rfc < 0 || rterm || rnc <= 0 || slot >= rnc) && node1 >= 0 &&
            node1 < T.M) {
            const ChildRec r1 = load_rec(T, g0 + node1);
            if (r1.nc <= 64 * kKidRegs) {
                select_slot_cached(T, g0, node1, r1, g, B, c, C, rounds, c_puct, O, lane);
                return;
            }
        }
    }
    for (int64_t k = dup ? 0 : c; k < rounds; k += dup ? 1 : C) {
        const int64_t sim = k * B + g;
        int cand = (int)(k % C);
        if (!active) { empty_sim_rows(O, sim, lane); continue; }
        int slot = C <= 64 ? __shfl(lane_slot, cand, 64) : root_slots[g * C + cand];
        if (slot < 0 || slot >= max_root) { empty_sim_rows(O, sim, lane); continue; }
        if (rfc < 0 || rterm || rnc <= 0 || slot >= rnc) { empty_sim_rows(O, sim, lane); continue; }
        int node = rfc + slot;
        if (node < 0 || node >= T.M) { empty_sim_rows(O, sim, lane); continue; }
        int plen = 0, vlen = 0;
        const ChildRec r = load_rec(T, g0 + node);
        int pvc = r.vc;
        if (!det) {
            enter_rec(T, g0, node, r, false, 0.0f, O, sim, plen, vlen, lane);
            pvc = r.vc + 1;
        } else {  // the root child gets no penalty in this mode, only the path record
            if (lane == 0) {
                uint16_t* dst = reinterpret_cast<uint16_t*>(O.paths + sim * kDepth * 6);
                dst[0] = r.mb0;
                dst[1] = r.mb1;
                dst[2] = r.mb2;
            }
            plen = 1;
        }
        node = descend_rec(T, g0, node, r, pvc, 1, c_puct, det, sigma, q_penalty, O, sim, plen, vlen, lane);
        __syncthreads();  // the next simulation reads this one's statistics
        // the simulation's outputs go after the fence: nothing in this kernel
        // reads them, so their stores complete while the next one descends
        if (lane == 0) {
            O.leaf[sim] = node;
            O.plen[sim] = plen;
            O.vlen[sim] = vlen;
        }
        zero_tails(O, sim, plen, vlen, lane);
    }
}

// mcts_select_with_root_mask_kernel (mcts_tree.cuh:689-800), one wave per game
__global__ __launch_bounds__(64) void k_select_mask(Tree T, const int8_t* __restrict__ game_active,
                                                    const int32_t* __restrict__ root_nodes,
                                                    const int8_t* __restrict__ alive, int max_root, float c_puct,
                                                    int64_t B, int64_t total, int det, float sigma, float q_penalty,
                                                    SelectOut O) {
    const int64_t g = blockIdx.x;
    const int lane = threadIdx.x;
    if (g >= B) return;
    const int64_t g0 = g * T.M;
    for (int64_t sim = g; sim < total; sim += B) {
        if (!game_active[g]) { empty_sim_rows(O, sim, lane); continue; }
        int root = root_nodes[g];
        int node = root;
        int plen = 0, vlen = 0;
        int64_t ri = g0 + root;
        ChildRec rr = load_rec(T, ri);  // the root's record (its children, visits)
        const int fc = rr.fc, nc = rr.nc;
        bool go = !(fc < 0 || rr.it || nc == 0) && !(nc <= 0 || nc > 1024);
        int first_iter = 0;
        int pvc = rr.vc;
        if (go) {  // root level: PUCT over alive children
            float bs = -INFINITY;
            int bi = 0x7fffffff;
            ChildRec mine = rr;
            for (int c = lane; c < nc; c += 64) {
                int child = fc + c;
                if (child < 0 || child >= T.M) break;
                if (c >= max_root || !alive[g * max_root + c]) continue;
                ChildRec cr = load_rec(T, g0 + child);
                float sc = puct_rec(cr, pvc, c_puct);
                if (sc > -1e30f && (sc > bs || (sc == bs && c < bi))) {
                    bs = sc;
                    bi = c;
                    mine = cr;
                }
            }
            int c = wave_argmax_first(bs, bi);
            if (c >= 0) {
                node = fc + c;
                rr = shfl_rec(mine, c & 63);
                enter_rec(T, g0, node, rr, false, 0.0f, O, sim, plen, vlen, lane);
                pvc = rr.vc + 1;
                first_iter = 1;
            } else {
                go = false;
            }
        }
        if (go) node = descend_rec(T, g0, node, rr, pvc, first_iter, c_puct, det, sigma, q_penalty, O, sim, plen,
                                   vlen, lane);
        __syncthreads();  // the next simulation reads this one's statistics; outputs after the fence
        if (lane == 0) {
            O.leaf[sim] = node;
            O.plen[sim] = plen;
            O.vlen[sim] = vlen;
        }
        zero_tails(O, sim, plen, vlen, lane);
    }
}

// mcts_replay_kernel (mcts_tree.cuh:298-320): leaf = root + path moves.  One
// wave per simulation; the row is assembled in LDS and written once.  With
// `results`, also the leaf's stored result byte (the check_results_kernel
// pass of game_logic.cu:1239-1241 over the replayed rows; 0 for a zero row).
__global__ __launch_bounds__(64) void k_replay(const uint8_t* __restrict__ roots, int64_t B,
                                               uint8_t* __restrict__ leaves, const uint8_t* __restrict__ paths,
                                               const int32_t* __restrict__ plen, const int32_t* __restrict__ leaf_idx,
                                               int64_t total, int zero_idle, int32_t* __restrict__ results) {
    __shared__ uint4 row[kStateBytes / 16];
    const int64_t sim = blockIdx.x;
    const int lane = threadIdx.x;
    if (sim >= total) return;
    if (leaf_idx[sim] < 0) {
        if (zero_idle) {
            uint4* dst = reinterpret_cast<uint4*>(leaves + sim * kStateBytes);
            const uint4 z = make_uint4(0u, 0u, 0u, 0u);
            for (int i = lane; i < kStateBytes / 16; i += 64) dst[i] = z;
            if (results && lane == 0) results[sim] = 0;
        }
        return;
    }
    const uint4* src = reinterpret_cast<const uint4*>(roots + (sim % B) * kStateBytes);
    for (int i = lane; i < kStateBytes / 16; i += 64) row[i] = src[i];
    __syncthreads();
    if (lane == 0) {
        RowView v{reinterpret_cast<uint8_t*>(row)};
        int n = plen[sim];
        const uint8_t* p = paths + sim * kDepth * 6;
        for (int d = 0; d < n && d < kDepth; d++, p += 6) v.apply(p[0], p[1], p[2] | (p[3] << 8), p[4] | (p[5] << 8));
    }
    __syncthreads();
    uint4* dst = reinterpret_cast<uint4*>(leaves + sim * kStateBytes);
    for (int i = lane; i < kStateBytes / 16; i += 64) dst[i] = row[i];
    if (results && lane == 0) results[sim] = reinterpret_cast<const uint8_t*>(row)[OFF_RESULT];
}

// The replay (k_replay with its results) and the leaf rows' legal lists +
// features (k_legal<moves, features>) of a simulation wave in one launch,
// two simulations per workgroup (lane groups of 32, as k_legal): a group
// copies the root's row to the leaf row and loads the root's board into LDS
// (a zero row and board for an idle simulation), one lane applies the path
// to the board and writes each move's changed bytes into the leaf row
// (apply_mirrored; the path's moves staged in LDS 32 at a time), and the
// position program then runs on the board as it stands -- no second load.
__device__ __attribute__((aligned(16))) const uint8_t kZeroState[kStateBytes] = {};

__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(6))) void k_replay_legal(
    const uint8_t* __restrict__ roots, int64_t B, uint8_t* __restrict__ leaves, const uint8_t* __restrict__ paths,
    const int32_t* __restrict__ plen, const int32_t* __restrict__ leaf_idx, int64_t T, int32_t* __restrict__ results,
    uint8_t* __restrict__ moves_out, int32_t* __restrict__ n_out, float* __restrict__ feat_out) {
    __shared__ Pos PS[kPosPerWave];
    const int grp = threadIdx.x >> 5, l = threadIdx.x & 31;
    Pos& P = PS[grp];
    const int64_t i = (int64_t)blockIdx.x * kPosPerWave + grp;
    const bool live = i < T;
    const int64_t sim = live ? i : T - 1;  // a group past the end reads the last row and writes nothing
    const bool idle = leaf_idx[sim] < 0;
    const uint8_t* src = idle ? kZeroState : roots + (sim % B) * kStateBytes;
    uint8_t* leaf_row = leaves + sim * kStateBytes;
    if (live) {
        const uint4* s4 = reinterpret_cast<const uint4*>(src);
        uint4* d4 = reinterpret_cast<uint4*>(leaf_row);
        for (int k = l; k < kStateBytes / 16; k += 32) d4[k] = s4[k];
    }
    load_position(P, src, threadIdx.x);
    // the board, and the leaf row's copy before the lane applying the path
    // reads it back (the barrier's workgroup-scope fences; a device-scope
    // fence would write back the whole L2 on every workgroup)
    __syncthreads();
    const int n = live && !idle ? min(plen[sim], kDepth) : 0;
    static_assert(kPool >= 3 * kW, "the pool holds one staged path move per lane");
    uint16_t* stage = P.u2.pool;  // free until generation: 32 path moves as 3 half-words each
    for (int d0 = 0; d0 < n; d0 += kW) {
        if (d0 + l < n) {
            const uint16_t* m = reinterpret_cast<const uint16_t*>(paths + (sim * kDepth + d0 + l) * 6);
            const uint16_t a = m[0], b = m[1], c = m[2];
            stage[3 * l] = a;
            stage[3 * l + 1] = b;
            stage[3 * l + 2] = c;
        }
        hw_group_lockstep();
        if (l == 0) {
            const int e = min(n - d0, kW);
            for (int k = 0; k < e; k++) {
                const int a = stage[3 * k];
                apply_mirrored(P, leaf_row, a & 0xFF, a >> 8, stage[3 * k + 1], stage[3 * k + 2]);
            }
        }
        hw_group_lockstep();
    }
    __syncthreads();  // the board after the path; the leaf row's changed bytes
    if (live && l == 0) results[sim] = idle ? 0 : P.result;
    // legal lists end at their lengths: the wave's readers (successor rows,
    // expansion) stop there
    run_legal_loaded<true, true, false>(P, leaf_row, threadIdx.x, live ? moves_out + sim * (kMaxLegal * 6) : nullptr,
                                        live ? n_out + sim : nullptr, live ? feat_out + sim * kFeat : nullptr,
                                        nullptr, false);
}

// centroid of a state row (compute_centroid, state_encoder.cuh:889-906)
HW_INL void row_centroid(const uint8_t* __restrict__ S, int lane, int& cq, int& cr) {
    int q = 0, r = 0, n = 0;
    if (lane < 18) {
        uint32_t w = reinterpret_cast<const uint32_t*>(S + OFF_OCC)[lane];
        while (w) {
            int c = lane * 32 + __ffs(w) - 1;
            w &= w - 1;
            int row = row_of(c);
            q += c - row * kGrid - kHalf;
            r += row - kHalf;
            n++;
        }
    }
    int sq = wave_sum(q), sr = wave_sum(r), sn = wave_sum(n);
    cq = sn ? round_half_even_div(sq, sn) : 0;
    cr = sn ? round_half_even_div(sr, sn) : 0;
}

// result_to_value (mcts_tree.cuh:182-188)
__device__ __forceinline__ float result_value(int result, int turn) {
    if (result == 3) return 0.0f;
    int player = turn & 1;
    if (result == 1) return player == 0 ? 1.0f : -1.0f;
    if (result == 2) return player == 0 ? -1.0f : 1.0f;
    return 0.0f;
}

struct LeafIn {
    const int32_t* leaf;
    const uint8_t* states;
    const uint8_t* legal;
    const int32_t* nlegal;
    const float* priors;
    const float* childq;
    const int32_t* results;
};

// Expansion of one simulation's leaf (mcts_expand_dense_priors_kernel
// :971-1062 body); returns 1 when this simulation created the children.
HW_INL int expand_leaf(const Tree& T, int64_t g, int64_t sim, const LeafIn& L, int lane) {
    const int64_t g0 = g * T.M;
    const int leaf = L.leaf[sim];
    const int64_t li = g0 + leaf;
    const uint8_t* S = L.states + sim * kStateBytes;
    // every value the decision needs, loaded together (one memory round trip)
    const int res = L.results[sim];
    const int fc = T.fc[li];
    const int n = L.nlegal[sim];
    const int base = T.cnt[g];
    if (res != 0) {
        if (lane == 0) {
            T.it[li] = 1;
            T.tval[li] = result_value(res, S[OFF_TURN] | (S[OFF_TURN + 1] << 8));
        }
        __syncthreads();
        return 0;
    }
    if (fc != -1) return 0;
    if (n <= 0) return 0;
    if ((int64_t)base + n > T.M) return 0;  // pool exhausted: leaf stays unexpanded
    int cq, cr;
    row_centroid(S, lane, cq, cr);
    const uint8_t* mv = L.legal + sim * (kMaxLegal * 6);
    const float* pri = L.priors + sim * kMaxLegal;
    const float* cqv = L.childq + sim * kMaxLegal;
    for (int m = lane; m < n; m += 64) {
        const uint8_t* x = mv + 6 * m;
        int64_t ci = g0 + base + m;
        T.vc[ci] = 0;
        T.tv[ci] = 0.0f;
        T.pr[ci] = pri[m];
        T.pa[ci] = leaf;
        T.ai[ci] = move_action(x[0], x[1], x[2] | (x[3] << 8), x[4] | (x[5] << 8), cq, cr);
        T.fc[ci] = -1;
        T.nc[ci] = 0;
        T.it[ci] = 0;
        T.tval[ci] = 0.0f;
        T.ciq[ci] = cqv[m];
        uint8_t* d = T.mb + ci * 6;
        for (int b = 0; b < 6; b++) d[b] = x[b];
    }
    if (lane == 0) {
        T.cnt[g] = base + n;
        T.nc[li] = n;
        T.fc[li] = base;
    }
    __syncthreads();
    return 1;
}

__global__ __launch_bounds__(64) void k_expand(Tree T, LeafIn L, int64_t B, int64_t total,
                                               int8_t* __restrict__ was_expanded) {
    const int64_t g = blockIdx.x;
    const int lane = threadIdx.x;
    if (g >= B) return;
    for (int64_t sim = g; sim < total; sim += B) {
        int e = 0;
        if (L.leaf[sim] >= 0) e = expand_leaf(T, g, sim, L, lane);
        if (lane == 0) was_expanded[sim] = (int8_t)e;
    }
}

// centroid of the occupied cells from the 18 bitboard words held by lanes
// 0-17 (compute_centroid, state_encoder.cuh:889-906); wave-uniform result
HW_INL void words_centroid(uint32_t w, int lane, int& cq, int& cr) {
    int q = 0, r = 0, n = 0;
    while (w) {
        int c = lane * 32 + __ffs(w) - 1;
        w &= w - 1;
        int row = row_of(c);
        q += c - row * kGrid - kHalf;
        r += row - kHalf;
        n++;
    }
    int sq = wave_sum(q), sr = wave_sum(r), sn = wave_sum(n);
    cq = sn ? round_half_even_div(sq, sn) : 0;
    cr = sn ? round_half_even_div(sr, sn) : 0;
}

// One simulation of mcts_expand_and_backprop_dense_priors_kernel
// (mcts_tree.cuh:1068-1187), run by the whole wave.  A simulation's loads come
// in three dependent batches: its inputs (leaf, result, legal count, path,
// value, the leaf's bitboards, legal list, priors and child values), then the
// tree state they index (the leaf's children and terminal fields, the path
// nodes' statistics, the root above the path), then the root's statistics.
// Expansion and backup are stores; the caller's fence between simulations
// makes them visible to the next.
//
// kPlanned = false: the game's simulations in order on one wave; `cnt` is the
//   game's running node counter and the backup walks up to the root.
// kPlanned = true: one root child's simulations (k_eb_game): the expansion
//   decision and node base come from the plan (`planned` >= 0: expand at that
//   node id), the node counter and the root belong to the plan, so the walk
//   above the path stops below the root; only selection paths get here.
template <bool kPlanned>
HW_INL void eb_sim(const Tree& T, const LeafIn& L, const float* __restrict__ nn_values,
                   const int32_t* __restrict__ vl_paths, const int32_t* __restrict__ vl_lens, float q_penalty,
                   int64_t g, int64_t sim, int lane, int& cnt, int planned) {
    const int64_t g0 = g * T.M;
    const int leaf = L.leaf[sim];
    // first loads: the simulation's inputs (this kernel never writes them)
    const int res = L.results[sim];
    const int nl = L.nlegal[sim];
    int n = vl_lens[sim];
    n = n < 0 ? 0 : (n > kDepth ? kDepth : n);
    const float nn = nn_values[sim];
    const int32_t* vp = vl_paths + sim * kDepth;
    const int p0 = vp[lane], p1 = vp[64 + lane];  // a path row holds kDepth = 128 entries
    const uint8_t* S = L.states + sim * kStateBytes;
    const int turn = S[OFF_TURN] | (S[OFF_TURN + 1] << 8);
    const uint32_t occw = lane < 18 ? reinterpret_cast<const uint32_t*>(S + OFF_OCC)[lane] : 0u;
    const uint8_t* mv = L.legal + sim * (kMaxLegal * 6);
    const float* pri = L.priors + sim * kMaxLegal;
    const float* cqv = L.childq + sim * kMaxLegal;
    uint16_t x0[4], x1[4], x2[4];
    float xp[4], xq[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int m = lane + 64 * j;
        x0[j] = x1[j] = x2[j] = 0;
        xp[j] = xq[j] = 0.0f;
        if (m < nl) {
            const uint16_t* x = reinterpret_cast<const uint16_t*>(mv + 6 * m);
            x0[j] = x[0];
            x1[j] = x[1];
            x2[j] = x[2];
            xp[j] = pri[m];
            xq[j] = cqv[m];
        }
    }
    // second loads: the tree state they index
    const int64_t li = g0 + leaf;
    const int fc = T.fc[li];
    const int lit = T.it[li];
    const float ltv = T.tval[li];
    const int last = n > 0 ? __shfl(n - 1 < 64 ? p0 : p1, (n - 1) & 63, 64) : leaf;
    // The selection entered vp[0..n) below the root, each node a child of
    // the one before, so the backup chain leaf -> root is that path
    // reversed, then the root; the expansion below writes none of them.
    // A path that ends at the leaf but is not such a chain (an entry outside
    // the pool, or one whose parent is not the entry before it) takes the
    // reference's serial walk instead: the parent links load beside the
    // statistics, and lane 0's is the node above the path.
    const bool in0 = lane < n && p0 >= 0 && p0 < T.M;
    const bool in1 = lane + 64 < n && p1 >= 0 && p1 < T.M;
    const bool maybe = last == leaf && __ballot((lane < n && !in0) || (lane + 64 < n && !in1)) == 0ull;
    int vc0 = 0, vc1 = 0, pa0 = -1, pa1 = -1;
    float tv0 = 0.0f, tv1 = 0.0f, vq0 = 0.0f, vq1 = 0.0f;
    if (maybe) {
        if (in0) {
            const int64_t ni = g0 + p0;
            tv0 = T.tv[ni];
            vc0 = T.vc[ni];
            vq0 = T.vq[ni];
            pa0 = T.pa[ni];
        }
        if (in1) {
            const int64_t ni = g0 + p1;
            tv1 = T.tv[ni];
            vc1 = T.vc[ni];
            vq1 = T.vq[ni];
            pa1 = T.pa[ni];
        }
    }
    const int prev0 = __shfl(p0, (lane + 63) & 63, 64);  // vp[lane - 1] (lane > 0)
    const int p0_63 = __shfl(p0, 63, 64);
    const int p1_up = __shfl(p1, (lane + 63) & 63, 64);
    const int prev1 = lane == 0 ? p0_63 : p1_up;  // vp[lane + 63]
    const bool broken = (in0 && lane > 0 && pa0 != prev0) || (in1 && pa1 != prev1);
    const bool chain = maybe && __ballot(broken) == 0ull;
    const int top = (chain && n > 0) ? __shfl(pa0, 0, 64) : leaf;  // the node above the path
    // expansion (mcts_expand_dense_priors_kernel :971-1062 body)
    int e = 0;
    float rv = 0.0f;
    const bool grow = kPlanned ? (res == 0 && planned >= 0)
                               : (res == 0 && fc == -1 && nl > 0 && (int64_t)cnt + nl <= T.M);
    const int base = kPlanned ? planned : cnt;
    if (res != 0) {
        rv = result_value(res, turn);
        if (lane == 0) {
            T.it[li] = 1;
            T.tval[li] = rv;
        }
    } else if (grow) {
        int cq, cr;
        words_centroid(occw, lane, cq, cr);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int m = lane + 64 * j;
            if (m >= nl) break;
            const int64_t ci = g0 + base + m;
            T.vc[ci] = 0;
            T.tv[ci] = 0.0f;
            T.pr[ci] = xp[j];
            T.pa[ci] = leaf;
            T.ai[ci] = move_action(x0[j] & 0xFF, x0[j] >> 8, x1[j], x2[j], cq, cr);
            T.fc[ci] = -1;
            T.nc[ci] = 0;
            T.it[ci] = 0;
            T.tval[ci] = 0.0f;
            T.ciq[ci] = xq[j];
            uint16_t* d = reinterpret_cast<uint16_t*>(T.mb + ci * 6);
            d[0] = x0[j];
            d[1] = x1[j];
            d[2] = x2[j];
        }
        for (int m = lane + 256; m < nl; m += 64) {  // lists beyond 256 entries (never produced here)
            const uint8_t* x = mv + 6 * m;
            const int64_t ci = g0 + base + m;
            T.vc[ci] = 0;
            T.tv[ci] = 0.0f;
            T.pr[ci] = pri[m];
            T.pa[ci] = leaf;
            T.ai[ci] = move_action(x[0], x[1], x[2] | (x[3] << 8), x[4] | (x[5] << 8), cq, cr);
            T.fc[ci] = -1;
            T.nc[ci] = 0;
            T.it[ci] = 0;
            T.tval[ci] = 0.0f;
            T.ciq[ci] = cqv[m];
            uint8_t* d = T.mb + ci * 6;
            for (int b = 0; b < 6; b++) d[b] = x[b];
        }
        if (lane == 0) {
            if (!kPlanned) T.cnt[g] = base + nl;
            T.nc[li] = nl;
            T.fc[li] = base;
        }
        if (!kPlanned) cnt += nl;
        e = 1;
    }
    const float v = res != 0 ? rv : (lit ? ltv : (e ? nn : 0.0f));
    if (chain) {  // each path node: virtual-loss undo, then the value; lanes side by side
        if (lane < n) {
            const int64_t ni = g0 + p0;
            const float sv = ((n - 1 - lane) & 1) ? -v : v;
            if (q_penalty > 0.0f) {
                T.vq[ni] = vq0 + -q_penalty;
                T.vc[ni] = vc0 + 1;
                T.tv[ni] = tv0 + sv;
            } else {  // visits -1 then +1; value +1.0 then the backed-up value
                T.tv[ni] = (tv0 + 1.0f) + sv;
            }
        }
        if (lane + 64 < n) {
            const int64_t ni = g0 + p1;
            const float sv = ((n - 1 - (lane + 64)) & 1) ? -v : v;
            if (q_penalty > 0.0f) {
                T.vq[ni] = vq1 + -q_penalty;
                T.vc[ni] = vc1 + 1;
                T.tv[ni] = tv1 + sv;
            } else {
                T.tv[ni] = (tv1 + 1.0f) + sv;
            }
        }
        if (lane == 0) {  // third loads: the nodes above the path (below the root when planned)
            int node = top;
            float w = (n & 1) ? -v : v;
            for (int s2 = n; s2 < kDepth + 1 && node >= 0; s2++) {
                const int64_t ni = g0 + node;
                const int up = T.pa[ni];
                if (kPlanned && up < 0) break;  // the root: the plan's
                T.vc[ni] += 1;
                T.tv[ni] += w;
                w = -w;
                node = up;
            }
        }
    } else if (!kPlanned && lane == 0) {  // not a selection path: the reference's serial walk
        for (int k = 0; k < n; k++) {
            const int64_t ni = g0 + vp[k];
            if (q_penalty > 0.0f) {
                T.vq[ni] += -q_penalty;
            } else {
                T.vc[ni] -= 1;
                T.tv[ni] += 1.0f;
            }
        }
        float w = v;
        int node = leaf;
        for (int s2 = 0; s2 < kDepth + 1 && node >= 0; s2++) {
            const int64_t ni = g0 + node;
            T.vc[ni] += 1;
            T.tv[ni] += w;
            w = -w;
            node = T.pa[ni];
        }
    }
}

// mcts_expand_and_backprop_dense_priors_kernel (mcts_tree.cuh:1068-1187):
// one wave per game, the game's simulations in order.
__global__ __launch_bounds__(64) void k_expand_backprop(Tree T, LeafIn L, const float* __restrict__ nn_values,
                                                        const int32_t* __restrict__ vl_paths,
                                                        const int32_t* __restrict__ vl_lens, float q_penalty,
                                                        int64_t B, int64_t total) {
    const int64_t g = blockIdx.x;
    const int lane = threadIdx.x;
    if (g >= B) return;
    int cnt = T.cnt[g];  // the game's node counter: only this wave changes it during the kernel
    for (int64_t sim = g; sim < total; sim += B) {
        if (L.leaf[sim] < 0) continue;
        eb_sim<false>(T, L, nn_values, vl_paths, vl_lens, q_penalty, g, sim, lane, cnt, -1);
        __syncthreads();  // the next simulation reads this one's stores
    }
}

// The same kernel over root children.  Below the root, a simulation touches
// only the subtree of the root child it entered: its path, its leaf and the
// leaf's new children.  So the simulations of different root children are
// independent except for two things a planning wave settles first, in
// simulation order: node ids (an exclusive prefix sum of the expansion sizes)
// and the root's statistics.  Then each root child's simulations are applied
// in order by one wave, with the same float operations in the same order per
// node as the one-wave kernel.  Games where this does not hold -- the node
// pool could run short, a path that is not a selection path, a leaf at the
// root -- are flagged, and the game's first wave runs all its simulations in
// order instead.  One workgroup per game (k_eb_game): wave 0 plans into LDS,
// one workgroup barrier, then wave w applies root-child groups w, w + waves,
// ...
constexpr int kPlanMax = 64;  // simulations per game one planning wave takes (one per lane)
constexpr int kEbWaves = 16;  // waves of a game's workgroup (at most kPlanMax groups, looped)

struct EbPlan {
    int base[kPlanMax];   // node id of simulation k's first new child, -1 = none
    int group[kPlanMax];  // root-child group of simulation k, -1 = idle
    int ngroups;
    int sequential;       // 1 = the game runs in the one-wave order
};

// The planning wave of game g (its simulations k * B + g, k < K, one per lane).
HW_INL void eb_plan_game(const Tree& T, const LeafIn& L, const float* __restrict__ nn_values,
                         const int32_t* __restrict__ vl_paths, const int32_t* __restrict__ vl_lens, int64_t B,
                         int64_t total, int64_t g, int lane, EbPlan& P) {

    const int K = (int)(total / B);  // the host launches this only for total = K * B, K <= kPlanMax
    const int64_t g0 = g * T.M;
    const int64_t sim = (int64_t)lane * B + g;
    const int cnt0 = T.cnt[g];
    int leaf = -1;
    if (lane < K) leaf = L.leaf[sim];
    const bool live = leaf >= 0;
    int res = 0, nl = 0, n = 0, fc0 = -1, lit = 0, turn = 0, top = -1, x = -1, head = -1;
    float ltv = 0.0f, nn = 0.0f;
    bool chain = true;
    if (live) {  // loads in dependent rounds: the simulation's inputs (with the path's first 8
                 // entries), then the path nodes' parents, then the walk above the path
        const int32_t* vp = vl_paths + sim * kDepth;
        int pv[8];
#pragma unroll
        for (int k = 0; k < 8; k++) pv[k] = vp[k];  // a path row holds kDepth = 128 entries
        res = L.results[sim];
        nl = L.nlegal[sim];
        n = vl_lens[sim];
        nn = nn_values[sim];
        const uint8_t* S = L.states + sim * kStateBytes;
        turn = S[OFF_TURN] | (S[OFF_TURN + 1] << 8);
        fc0 = T.fc[g0 + leaf];
        lit = T.it[g0 + leaf];
        ltv = T.tval[g0 + leaf];
        n = n < 0 ? 0 : (n > kDepth ? kDepth : n);
        // a selection path: every entry in the pool, each the child of the entry
        // before, the last one the leaf (eb_sim's chain test, which the planned waves rely on)
        head = n > 0 ? pv[0] : leaf;
        top = leaf;
        x = leaf;
        int prev = -1;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            if (k < n) {
                const int e = pv[k];
                if (e < 0 || e >= T.M) {
                    chain = false;
                } else {
                    const int up = T.pa[g0 + e];
                    if (k == 0) top = up;
                    else if (up != prev) chain = false;
                }
                prev = e;
                x = e;
            }
        }
        for (int k = 8; k < n && chain; k++) {  // longer paths, entry by entry
            const int e = vp[k];
            if (e < 0 || e >= T.M || T.pa[g0 + e] != prev) chain = false;
            prev = e;
            x = e;
        }
    }
    bool bad = live && (!chain || x != leaf);
    // the walk above the path: top, its parent, ... up to the root (parent -1)
    int root = -1, steps = 0, key = head;
    if (live && !bad) {
        int node = top, below = head, up = top >= 0 ? T.pa[g0 + top] : -1;
        while (node >= 0 && up >= 0 && steps < kDepth + 1) {
            below = node;
            node = up;
            up = T.pa[g0 + node];
            steps++;
        }
        root = node;
        key = below;  // the root child the simulation went through
        if (node < 0 || up >= 0 || key == root) bad = true;  // no root within reach, or the leaf is the root
    }
    // expansion sizes: the first simulation reaching an unexpanded leaf expands it
    bool first = live;
    for (int k = 0; k < K; k++) {  // k is wave-uniform: lane values by readlane (no LDS round trip)
        const int lk = __builtin_amdgcn_readlane(leaf, k);
        if (k < lane && lk == leaf) first = false;
    }
    const int sz = (live && res == 0 && fc0 == -1 && nl > 0 && first) ? nl : 0;
    const int pre = wave_excl_scan(sz, lane);
    const int tot = wave_sum(sz);
    const bool seq = __ballot(bad) != 0ull || (int64_t)cnt0 + tot > T.M;
    // root-child groups in order of first appearance
    int firstk = lane;
    const uint64_t livem = __ballot(live);
    for (int k = K - 1; k >= 0; k--) {
        const int kk = __builtin_amdgcn_readlane(key, k);
        if (k < lane && ((livem >> k) & 1ull) && kk == key) firstk = k;
    }
    const bool opens = live && firstk == lane;
    const uint64_t om = __ballot(opens);
    const int gid_own = __popcll(om & ((1ull << lane) - 1ull));
    const int gid = __shfl(gid_own, firstk, 64);
    if (lane < K) {
        P.base[lane] = (!seq && sz > 0) ? cnt0 + pre : -1;
        P.group[lane] = (!seq && live) ? gid : -1;
    }
    if (lane == 0) {
        P.ngroups = seq ? 0 : __popcll(om);
        P.sequential = seq ? 1 : 0;
        if (!seq) T.cnt[g] = cnt0 + tot;
    }
    if (seq) return;
    // the root's statistics, in simulation order: +1 visit and the value with the
    // sign it has at the root (alternating per level from the leaf)
    const float v = res != 0 ? result_value(res, turn) : (lit ? ltv : (sz > 0 ? nn : 0.0f));
    const float wtop = (n & 1) ? -v : v;
    const float wroot = (steps & 1) ? -wtop : wtop;
    const bool hits = live && n + steps < kDepth + 1;  // the walk's bound (as k_expand_backprop)
    // (the loop runs on the whole wave, so the shuffles read active lanes; lane 0
    // holds the accumulators and does the memory accesses)
    int cur = -1, vcn = 0;
    float tvn = 0.0f;
    const uint64_t hitm = __ballot(hits);
    for (int k = 0; k < K; k++) {
        if (!((hitm >> k) & 1ull)) continue;
        const int r = __builtin_amdgcn_readlane(root, k);
        const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wroot), k));
        if (r != cur) {
            if (cur >= 0 && lane == 0) {
                T.vc[g0 + cur] = vcn;
                T.tv[g0 + cur] = tvn;
            }
            cur = r;
            if (lane == 0) {
                vcn = T.vc[g0 + r];
                tvn = T.tv[g0 + r];
            }
        }
        vcn += 1;
        tvn += w;
    }
    if (cur >= 0 && lane == 0) {
        T.vc[g0 + cur] = vcn;
        T.tv[g0 + cur] = tvn;
    }
}

__global__ __launch_bounds__(64 * kEbWaves) void k_eb_game(Tree T, LeafIn L, const float* __restrict__ nn_values,
                                                          const int32_t* __restrict__ vl_paths,
                                                          const int32_t* __restrict__ vl_lens, float q_penalty,
                                                          int64_t B, int64_t total) {
    __shared__ EbPlan P;
    const int64_t g = blockIdx.x;  // the grid is B workgroups
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, waves = blockDim.x >> 6;
    if (wave == 0) eb_plan_game(T, L, nn_values, vl_paths, vl_lens, B, total, g, lane, P);
    // the plan (LDS) and its tree writes (node count, root statistics) before
    // any wave applies; the only barrier of the kernel, reached by every wave
    __syncthreads();
    // Between two simulations of one wave a workgroup-scope fence orders the
    // first's stores before the second's loads (the lanes of a wave run in
    // step; no barrier, the waves' loop counts differ).
    if (P.sequential) {  // a game the plan left to the one-wave order: its first wave runs it
        if (wave != 0) return;
        int cnt = T.cnt[g];
        for (int64_t sim = g; sim < total; sim += B) {
            if (L.leaf[sim] < 0) continue;
            eb_sim<false>(T, L, nn_values, vl_paths, vl_lens, q_penalty, g, sim, lane, cnt, -1);
            __threadfence_block();
        }
        return;
    }
    const int K = (int)(total / B);
    const int plan = lane < K ? P.base[lane] : -1;
    const int grp = lane < K ? P.group[lane] : -1;
    const int ng = P.ngroups;
    for (int j = wave; j < ng; j += waves) {
        uint64_t m = __ballot(grp == j);
        int unused = 0;
        while (m) {
            const int k = __ffsll((unsigned long long)m) - 1;
            m &= m - 1;
            eb_sim<true>(T, L, nn_values, vl_paths, vl_lens, q_penalty, g, (int64_t)k * B + g, lane, unused,
                         __shfl(plan, k, 64));
            __threadfence_block();  // the next simulation of this root child reads this one's stores
        }
    }
}

// mcts_root_noise_kernel (mcts_tree.cuh:1192-1234), one lane per game
__global__ void k_root_noise(Tree T, const float* __restrict__ noise, const int32_t* __restrict__ root_nodes,
                             int pad, float eps, float temp, int64_t B) {
    int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= B) return;
    const int64_t g0 = g * T.M;
    int64_t ri = g0 + root_nodes[g];
    int fc = T.fc[ri], nc = T.nc[ri];
    if (fc < 0 || nc == 0) return;
    const float* z = noise + g * pad;
    if (temp > 1.0f) {
        float inv = 1.0f / temp, sum = 0.0f;
        for (int c = 0; c < nc; c++) {
            float p = powf(T.pr[g0 + fc + c], inv);
            T.pr[g0 + fc + c] = p;
            sum += p;
        }
        if (sum > 0.0f)
            for (int c = 0; c < nc; c++) T.pr[g0 + fc + c] /= sum;
    }
    if (eps > 0.0f) {
        for (int c = 0; c < nc && c < pad; c++) {
            float a = (1.0f - eps) * T.pr[g0 + fc + c];
            float b = eps * z[c];
            T.pr[g0 + fc + c] = a + b;
        }
    }
}

inline int finish() { return (int)hipGetLastError(); }


// Hard rebase of the games with reset[g] != 0 (_reroot_tree,
// fnn_mcts_orchestrator.py:1122-1142): the reference refills all max_nodes
// entries of the game's rows; nodes at or beyond node_count[g] have never
// been written since the game's last reset (expansion hands out ids below
// node_count only), so refilling the used prefix [0, node_count) gives the
// same arrays.  grid (x, B): the x blocks of game g stride over its prefix.
// node_count / root_node are reset by k_reset_counts after this kernel.
__global__ __launch_bounds__(256) void k_reset_nodes(Tree T, const int8_t* __restrict__ reset, int64_t B) {
    const int64_t g = blockIdx.y;
    if (g >= B || !reset[g]) return;
    int64_t cnt = T.cnt[g];
    cnt = cnt < 0 ? 0 : (cnt > T.M ? T.M : cnt);
    const int64_t base = g * T.M;
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < cnt; j += (int64_t)gridDim.x * blockDim.x) {
        const int64_t n = base + j;
        T.vc[n] = 0;
        T.tv[n] = 0.0f;
        T.pr[n] = 0.0f;
        T.pa[n] = -1;
        T.ai[n] = -1;
        T.fc[n] = -1;
        T.nc[n] = 0;
        T.it[n] = 0;
        T.tval[n] = 0.0f;
        T.ciq[n] = 0.0f;
        uint8_t* mb = T.mb + n * 6;
#pragma unroll
        for (int b = 0; b < 6; b++) mb[b] = 0;
    }
}

__global__ void k_reset_counts(int32_t* __restrict__ cnt, int32_t* __restrict__ root_node,
                               const int8_t* __restrict__ reset, int64_t B) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g < B && reset[g]) {
        cnt[g] = 1;
        root_node[g] = 0;
    }
}
// ---------------------------------------------------------------- legacy
// The action-space engine behind hive_gpu/gpu_native_mcts.py: PUCT from the
// root (no root slots or mask), priors looked up in [T][85834] action rows,
// a separate backup kernel and the [B][85834] visit policy.  Same canonical
// order as above: one wave per game, its simulations in order.
constexpr int kActions = 85834;

// mcts_select_kernel (mcts_tree.cuh:205-296): the first child stands when no
// score beats -1e30
__global__ __launch_bounds__(64) void k_select_legacy(Tree T, const int8_t* __restrict__ game_active,
                                                      const int32_t* __restrict__ root_nodes, float c_puct, int64_t B,
                                                      int64_t total, SelectOut O) {
    const int64_t g = blockIdx.x;
    const int lane = threadIdx.x;
    if (g >= B) return;
    const int64_t g0 = g * T.M;
    for (int64_t sim = g; sim < total; sim += B) {
        if (!game_active[g]) { empty_sim(O, sim, lane); continue; }
        int node = root_nodes[g];
        int plen = 0, vlen = 0;
        for (int it = 0; it < kDepth; it++) {
            int64_t ni = g0 + node;
            int cfc = T.fc[ni], cnc = T.nc[ni];
            if (cfc < 0 || T.it[ni] || cnc == 0) break;
            if (cnc <= 0 || cnc > 1024 || cfc >= T.M) break;
            float bs = -INFINITY;
            int bi = 0x7fffffff;
            for (int c = lane; c < cnc; c += 64) {
                int child = cfc + c;
                if (child < 0 || child >= T.M) break;
                float sc = puct(T, ni, g0 + child, c_puct);
                if (sc > -1e30f && (sc > bs || (sc == bs && c < bi))) { bs = sc; bi = c; }
            }
            int c = wave_argmax_first(bs, bi);
            node = cfc + (c < 0 ? 0 : c);
            enter(T, g0, node, false, 0.0f, O, sim, plen, vlen, lane);
        }
        if (lane == 0) {
            O.leaf[sim] = node;
            O.plen[sim] = plen;
            O.vlen[sim] = vlen;
        }
        __syncthreads();
    }
}

// mcts_expand_kernel (mcts_tree.cuh:330-433) body: a child per legal move with
// an action index (moves outside the 17x17 window are skipped), prior =
// action row[action]; virtual_q_penalty and child_init_q are not touched
HW_INL int expand_leaf_legacy(const Tree& T, int64_t g, int64_t sim, const LeafIn& L, int lane) {
    const int64_t g0 = g * T.M;
    int leaf = L.leaf[sim];
    int64_t li = g0 + leaf;
    const uint8_t* S = L.states + sim * kStateBytes;
    int res = L.results[sim];
    if (res != 0) {
        if (lane == 0) {
            T.it[li] = 1;
            T.tval[li] = result_value(res, S[OFF_TURN] | (S[OFF_TURN + 1] << 8));
        }
        __syncthreads();
        return 0;
    }
    if (T.fc[li] != -1) return 0;
    int n = L.nlegal[sim];
    n = n > kMaxLegal ? kMaxLegal : n;
    if (n <= 0) return 0;
    int base = T.cnt[g];
    if ((int64_t)base + n > T.M) return 0;
    int cq, cr;
    row_centroid(S, lane, cq, cr);
    const uint8_t* mv = L.legal + sim * (kMaxLegal * 6);
    const float* probs = L.priors + sim * (int64_t)kActions;
    int created = 0;
    for (int m0 = 0; m0 < n; m0 += 64) {
        const int m = m0 + lane;
        int a = -1;
        const uint8_t* x = mv + 6 * m;
        if (m < n) a = move_action(x[0], x[1], x[2] | (x[3] << 8), x[4] | (x[5] << 8), cq, cr);
        const uint64_t keep = __ballot(a >= 0);
        if (a >= 0) {
            int64_t ci = g0 + base + created + __popcll(keep & ((1ull << lane) - 1ull));
            T.vc[ci] = 0;
            T.tv[ci] = 0.0f;
            T.pr[ci] = probs[a];
            T.pa[ci] = leaf;
            T.ai[ci] = a;
            T.fc[ci] = -1;
            T.nc[ci] = 0;
            T.it[ci] = 0;
            T.tval[ci] = 0.0f;
            uint8_t* d = T.mb + ci * 6;
            for (int b = 0; b < 6; b++) d[b] = x[b];
        }
        created += __popcll(keep);
    }
    if (lane == 0) {
        T.cnt[g] = base + created;
        T.nc[li] = created;
        T.fc[li] = base;
    }
    __syncthreads();
    return 1;
}

// value backup of one simulation (mcts_backprop_kernel :555-605): virtual
// losses undone along its path, then +1 visit and the sign-alternating value
// from the leaf up the parent links
HW_INL void backup_sim(const Tree& T, int64_t g0, int64_t sim, int leaf, float v, const int32_t* __restrict__ vl_paths,
                       const int32_t* __restrict__ vl_lens) {
    int n = vl_lens[sim];
    const int32_t* vp = vl_paths + sim * kDepth;
    for (int k = 0; k < n && k < kDepth; k++) {
        int64_t ni = g0 + vp[k];
        T.vc[ni] -= 1;
        T.tv[ni] += 1.0f;
    }
    int node = leaf;
    for (int s = 0; s < kDepth + 1 && node >= 0; s++) {
        int64_t ni = g0 + node;
        T.vc[ni] += 1;
        T.tv[ni] += v;
        v = -v;
        node = T.pa[ni];
    }
}

__global__ __launch_bounds__(64) void k_expand_legacy(Tree T, LeafIn L, int64_t B, int64_t total,
                                                      int8_t* __restrict__ was_expanded) {
    const int64_t g = blockIdx.x;
    const int lane = threadIdx.x;
    if (g >= B) return;
    for (int64_t sim = g; sim < total; sim += B) {
        int e = 0;
        if (L.leaf[sim] >= 0) e = expand_leaf_legacy(T, g, sim, L, lane);
        if (lane == 0) was_expanded[sim] = (int8_t)e;
    }
}

__global__ __launch_bounds__(64) void k_backprop_legacy(Tree T, const int32_t* __restrict__ leaf_idx,
                                                        const float* __restrict__ nn_values,
                                                        const int32_t* __restrict__ vl_paths,
                                                        const int32_t* __restrict__ vl_lens,
                                                        const int8_t* __restrict__ was_expanded, int64_t B,
                                                        int64_t total) {
    const int64_t g = blockIdx.x;
    if (g >= B || threadIdx.x != 0) return;
    const int64_t g0 = g * T.M;
    for (int64_t sim = g; sim < total; sim += B) {
        int leaf = leaf_idx[sim];
        if (leaf < 0) continue;
        int64_t li = g0 + leaf;
        float v = T.it[li] ? T.tval[li] : (was_expanded[sim] ? nn_values[sim] : 0.0f);
        backup_sim(T, g0, sim, leaf, v, vl_paths, vl_lens);
    }
}

// mcts_expand_and_backprop_kernel (mcts_tree.cuh:435-553)
__global__ __launch_bounds__(64) void k_expand_backprop_legacy(Tree T, LeafIn L, const float* __restrict__ nn_values,
                                                               const int32_t* __restrict__ vl_paths,
                                                               const int32_t* __restrict__ vl_lens, int64_t B,
                                                               int64_t total) {
    const int64_t g = blockIdx.x;
    const int lane = threadIdx.x;
    if (g >= B) return;
    const int64_t g0 = g * T.M;
    for (int64_t sim = g; sim < total; sim += B) {
        int leaf = L.leaf[sim];
        if (leaf < 0) continue;
        int e = expand_leaf_legacy(T, g, sim, L, lane);
        if (lane == 0) {
            int64_t li = g0 + leaf;
            backup_sim(T, g0, sim, leaf, T.it[li] ? T.tval[li] : (e ? nn_values[sim] : 0.0f), vl_paths, vl_lens);
        }
        __syncthreads();
    }
}

// mcts_extract_policy_kernel (mcts_tree.cuh:607-687): the game's [85834] row
// is written whole (zeros, then the root children's values, serially in
// child order as the reference sums them)
__global__ __launch_bounds__(64) void k_extract_policy(Tree T, const int32_t* __restrict__ move_numbers,
                                                       const int32_t* __restrict__ root_nodes, float temperature,
                                                       int temp_drop, float pruning, int64_t B,
                                                       float* __restrict__ policies) {
    const int64_t g = blockIdx.x;
    const int lane = threadIdx.x;
    if (g >= B) return;
    float* pol = policies + g * (int64_t)kActions;
    for (int i = lane; i < kActions; i += 64) pol[i] = 0.0f;
    __syncthreads();
    if (lane != 0) return;
    const int64_t g0 = g * T.M;
    int64_t ri = g0 + root_nodes[g];
    int fc = T.fc[ri], nc = T.nc[ri];
    if (fc < 0 || nc == 0) return;
    float temp = move_numbers[g] >= temp_drop ? 0.0f : temperature;
    if (temp <= 0.0f) {
        int best_a = -1, best_v = -1;
        for (int c = 0; c < nc; c++) {
            int64_t ci = g0 + fc + c;
            int v = T.vc[ci];
            if (v > best_v) { best_v = v; best_a = T.ai[ci]; }
        }
        if (best_a >= 0 && best_a < kActions) pol[best_a] = 1.0f;
        return;
    }
    float max_v = 0.0f, sum = 0.0f;
    for (int c = 0; c < nc; c++) {
        float v = (float)T.vc[g0 + fc + c];
        if (v > max_v) max_v = v;
    }
    for (int c = 0; c < nc; c++) {
        int64_t ci = g0 + fc + c;
        float v = (float)T.vc[ci];
        if (pruning > 0.0f && max_v > 0.0f && v < max_v * pruning) v = 0.0f;
        if (temp != 1.0f) v = powf(v, 1.0f / temp);
        int a = T.ai[ci];
        if (a >= 0 && a < kActions) {
            pol[a] = v;
            sum += v;
        }
    }
    if (sum > 0.0f) {
        for (int c = 0; c < nc; c++) {
            int a = T.ai[g0 + fc + c];
            if (a >= 0 && a < kActions) pol[a] /= sum;
        }
    } else {
        float u = 1.0f / (float)nc;
        for (int c = 0; c < nc; c++) {
            int a = T.ai[g0 + fc + c];
            if (a >= 0 && a < kActions) pol[a] = u;
        }
    }
}

// Per-wave search counters: stats[0] += simulations that reached a leaf,
// [1] += their leaf legal counts, [2] += their virtual-loss path lengths,
// [3] += rows.  Each workgroup sums 1,024 rows and adds its partial sums
// with device atomics (integer sums: the order does not matter).
__global__ __launch_bounds__(1024) void k_wave_stats(const int32_t* __restrict__ leaf_idx,
                                                     const int32_t* __restrict__ num_legal,
                                                     const int32_t* __restrict__ vl_lens, int64_t total,
                                                     unsigned long long* __restrict__ stats) {
    __shared__ unsigned long long part[3][16];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t i = (int64_t)blockIdx.x * 1024 + tid;
    unsigned long long a = 0, b = 0, c = 0;
    if (i < total && leaf_idx[i] >= 0) {
        a = 1;
        b = (unsigned long long)(long long)num_legal[i];
        c = (unsigned long long)(long long)vl_lens[i];
    }
    for (int off = 32; off > 0; off >>= 1) {
        a += __shfl_xor(a, off);
        b += __shfl_xor(b, off);
        c += __shfl_xor(c, off);
    }
    if (lane == 0) { part[0][w] = a; part[1][w] = b; part[2][w] = c; }
    __syncthreads();
    if (tid < 3) {
        unsigned long long sum = 0;
        for (int k = 0; k < 16; k++) sum += part[tid][k];
        atomicAdd(&stats[tid], sum);
    } else if (tid == 3 && blockIdx.x == 0) {
        atomicAdd(&stats[3], (unsigned long long)total);
    }
}

// ---------------------------------------------------------------- Gumbel halving
// One decision of sequential halving (fnn_mcts_orchestrator.py:650-731: the
// torch work between rounds, and the final choice).  A candidate column of
// game g holds a root slot (-1 = none); its statistics are those of the root
// child in that slot (_gather_root_candidate_stats: N, and Q = -W / max(N, 1)
// when N > min_visits; both 0 for a slot outside the root's children).  With
// m the batch's largest candidate visit count, sigma = (c_visit + m) *
// c_scale and the column's score is base[g][slot] + sigma * Q (-1e30 for an
// empty column).  keep > 0: the columns ranked by score (descending, ties to
// the lower column), the first keep of them written to cand_out[g][0..keep),
// the first max(1, valid / 2) as their slots and the rest as -1; keep = 0:
// chosen[g] = max(slot of the first highest column, 0).  Each workgroup finds
// m itself (every candidate, from L2), then ranks the columns of its games,
// one game per segment of Cp lanes (Cp = C rounded up to a power of two, at
// most 64), by shuffles.
constexpr int kHalvThreads = 1024;
struct RootStat {
    int v;
    float q;
};
__device__ __forceinline__ RootStat root_slot_stat(const Tree& T, const int32_t* __restrict__ root_nodes,
                                                   int64_t g, int slot, int min_visits) {
    RootStat r{0, 0.0f};
    if (slot < 0) return r;
    const int64_t g0 = g * T.M;
    const int root = root_nodes[g];
    const int fc = T.fc[g0 + root], nc = T.nc[g0 + root];
    if (fc < 0 || slot >= nc) return r;
    int64_t idx = (int64_t)fc + slot;
    idx = idx < T.M ? idx : T.M - 1;
    const int v = T.vc[g0 + idx];
    r.v = v;
    if (v > min_visits) r.q = -T.tv[g0 + idx] / (float)(v > 1 ? v : 1);
    return r;
}

__global__ __launch_bounds__(kHalvThreads) void k_gumbel_halving(Tree T, const int32_t* __restrict__ root_nodes,
                                                                 const int32_t* __restrict__ cand, int C, int Cp,
                                                                 const float* __restrict__ base, float c_visit,
                                                                 float c_scale, int min_visits, int keep, int64_t B,
                                                                 int32_t* __restrict__ cand_out,
                                                                 int64_t* __restrict__ chosen) {
    __shared__ int wmax[kHalvThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63;
    // the batch's largest candidate visit count (0 when none)
    int mx = 0;
    const int64_t n = B * C;
#pragma unroll 4
    for (int64_t i = tid; i < n; i += kHalvThreads) mx = max(mx, root_slot_stat(T, root_nodes, i / C, cand[i],
                                                                                  min_visits).v);
    for (int o = 32; o > 0; o >>= 1) mx = max(mx, __shfl_xor(mx, o, 64));
    if (lane == 0) wmax[tid >> 6] = mx;
    __syncthreads();
    mx = 0;
#pragma unroll
    for (int k = 0; k < kHalvThreads / 64; k++) mx = max(mx, wmax[k]);
    const float sigma = (c_visit + (float)mx) * c_scale;
    // this workgroup's games: one per Cp-lane segment
    const int c = tid & (Cp - 1), seg0 = lane & ~(Cp - 1);
    const int64_t g = (int64_t)blockIdx.x * (kHalvThreads / Cp) + tid / Cp;
    const bool real = g < B && c < C;
    int slot = -1;
    float score = -1e30f;
    if (real) {
        slot = cand[g * C + c];
        if (slot >= 0) {
            const RootStat st = root_slot_stat(T, root_nodes, g, slot, min_visits);
            score = base[g * kMaxLegal + (slot < kMaxLegal ? slot : kMaxLegal - 1)] + sigma * st.q;
        }
    }
    int rank = 0;
    for (int j = 0; j < Cp; j++) {  // uniform trip count: every lane takes part in the shuffles
        const float sj = __shfl(score, seg0 + j, 64);
        if (j < C && (sj > score || (sj == score && j < c))) rank++;
    }
    const uint64_t segmask = Cp == 64 ? ~0ull : (((1ull << Cp) - 1ull) << seg0);
    const int nvalid = __popcll(__ballot(real && slot >= 0) & segmask);
    if (!real) return;
    if (keep > 0) {
        const int keep_n = nvalid / 2 > 1 ? nvalid / 2 : 1;
        if (rank < keep) cand_out[g * keep + rank] = rank < keep_n ? slot : -1;
    } else if (rank == 0) {
        chosen[g] = slot < 0 ? 0 : slot;
    }
}

}  // namespace

// hg_mcts_expand_backprop_dense_ws's launch with at most `groups` waves per
// game's workgroup (every root child the game's simulations entered gets a
// wave when there are at most that many; the waves loop otherwise): the
// simulation wave passes its candidate count, which bounds the root children
// it enters, so that a small round does not reserve sixteen waves per game.
static int eb_games(const hg_tree* tree, const float* child_q_values, const int32_t* leaf_idx,
                    const uint8_t* leaf_states, const uint8_t* legal_moves, const int32_t* num_legal,
                    const float* priors_per_legal, const int32_t* results, const float* nn_values,
                    const int32_t* vl_paths, const int32_t* vl_lens, float q_penalty, int64_t B, int64_t total,
                    int groups, hipStream_t stream) {
    if (B <= 0 || total <= 0) return 0;
    const int64_t K = total / B;
    if (total % B != 0 || K > kPlanMax || B * K > (int64_t)INT32_MAX)  // outside the planner's shape
        return hg_mcts_expand_backprop_dense(tree, child_q_values, leaf_idx, leaf_states, legal_moves, num_legal,
                                             priors_per_legal, results, nn_values, vl_paths, vl_lens, q_penalty, B,
                                             total, stream);
    LeafIn L{leaf_idx, leaf_states, legal_moves, num_legal, priors_per_legal, child_q_values, results};
    int64_t waves = K < kEbWaves ? K : kEbWaves;
    if (groups < waves) waves = groups < 1 ? 1 : groups;
    hipLaunchKernelGGL(k_eb_game, dim3((unsigned)B), dim3((unsigned)(64 * waves)), 0, stream, to_tree(tree), L,
                       nn_values, vl_paths, vl_lens, q_penalty, B, total);
    return finish();
}

// hg_mcts_select_root_slots with the path rows' tails zeroed or left
// (O.tails)
static int select_root_slots(const hg_tree* tree, const int8_t* game_active, const int32_t* root_nodes,
                             const int32_t* root_slots, int num_candidates, int max_root_children, float c_puct,
                             int64_t B, int W, int deterministic_non_root, float non_root_sigma, float q_penalty,
                             const SelectOut& O, hipStream_t stream) {
    if (B <= 0 || W <= 0 || num_candidates <= 0) return 0;
    const int64_t total = (int64_t)W * num_candidates * B;
    if (B * num_candidates > (int64_t)0x7fffffff) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_select_slots, dim3((unsigned)(B * num_candidates)), dim3(64), 0, stream, to_tree(tree),
                       game_active, root_nodes, root_slots, num_candidates, max_root_children, c_puct, B, total,
                       deterministic_non_root, non_root_sigma, q_penalty, O);
    return finish();
}

extern "C" {

int hg_mcts_wave_stats(const int32_t* leaf_idx, const int32_t* num_legal, const int32_t* vl_lens, int64_t total,
                       int64_t* stats, void* stream) {
    if (total <= 0) return 0;
    hipLaunchKernelGGL(k_wave_stats, dim3((unsigned)((total + 1023) / 1024)), dim3(1024), 0, (hipStream_t)stream,
                       leaf_idx, num_legal, vl_lens, total, reinterpret_cast<unsigned long long*>(stats));
    return finish();
}

int hg_mcts_select_root_slots(const hg_tree* tree, const int8_t* game_active, const int32_t* root_nodes,
                              const int32_t* root_slots, int num_candidates, int max_root_children, float c_puct,
                              int64_t B, int W, int deterministic_non_root, float non_root_sigma, float q_penalty,
                              int32_t* leaf_idx, uint8_t* move_paths, int32_t* path_lens, int32_t* vl_paths,
                              int32_t* vl_lens, void* stream) {
    return select_root_slots(tree, game_active, root_nodes, root_slots, num_candidates, max_root_children, c_puct, B,
                             W, deterministic_non_root, non_root_sigma, q_penalty,
                             SelectOut{leaf_idx, move_paths, path_lens, vl_paths, vl_lens, 1}, (hipStream_t)stream);
}

int hg_mcts_select_root_mask(const hg_tree* tree, const int8_t* game_active, const int32_t* root_nodes,
                             const int8_t* alive_mask, int max_root_children, float c_puct, int64_t B, int W,
                             int deterministic_non_root, float non_root_sigma, float q_penalty, int32_t* leaf_idx,
                             uint8_t* move_paths, int32_t* path_lens, int32_t* vl_paths, int32_t* vl_lens,
                             void* stream) {
    if (B <= 0 || W <= 0) return 0;
    int64_t total = (int64_t)W * B;
    SelectOut O{leaf_idx, move_paths, path_lens, vl_paths, vl_lens};
    hipLaunchKernelGGL(k_select_mask, dim3((unsigned)B), dim3(64), 0, (hipStream_t)stream, to_tree(tree),
                       game_active, root_nodes, alive_mask, max_root_children, c_puct, B, total,
                       deterministic_non_root, non_root_sigma, q_penalty, O);
    return finish();
}

int hg_mcts_replay(const uint8_t* root_states, int64_t B, uint8_t* leaf_states, const uint8_t* move_paths,
                   const int32_t* path_lens, const int32_t* leaf_idx, int64_t total, void* stream) {
    if (B <= 0 || total <= 0) return 0;
    hipLaunchKernelGGL(k_replay, dim3((unsigned)total), dim3(64), 0, (hipStream_t)stream, root_states, B,
                       leaf_states, move_paths, path_lens, leaf_idx, total, 0, nullptr);
    return finish();
}

int hg_mcts_replay_fill(const uint8_t* root_states, int64_t B, uint8_t* leaf_states, const uint8_t* move_paths,
                        const int32_t* path_lens, const int32_t* leaf_idx, int64_t total, void* stream) {
    if (B <= 0 || total <= 0) return 0;
    hipLaunchKernelGGL(k_replay, dim3((unsigned)total), dim3(64), 0, (hipStream_t)stream, root_states, B,
                       leaf_states, move_paths, path_lens, leaf_idx, total, 1, nullptr);
    return finish();
}

int hg_mcts_expand_dense(const hg_tree* tree, const float* child_q_values, const int32_t* leaf_idx,
                         const uint8_t* leaf_states, const uint8_t* legal_moves, const int32_t* num_legal,
                         const float* priors_per_legal, const int32_t* results, int64_t B, int64_t total,
                         int8_t* was_expanded, void* stream) {
    if (B <= 0 || total <= 0) return 0;
    LeafIn L{leaf_idx, leaf_states, legal_moves, num_legal, priors_per_legal, child_q_values, results};
    hipLaunchKernelGGL(k_expand, dim3((unsigned)B), dim3(64), 0, (hipStream_t)stream, to_tree(tree), L, B, total,
                       was_expanded);
    return finish();
}

int hg_mcts_expand_backprop_dense(const hg_tree* tree, const float* child_q_values, const int32_t* leaf_idx,
                                  const uint8_t* leaf_states, const uint8_t* legal_moves, const int32_t* num_legal,
                                  const float* priors_per_legal, const int32_t* results, const float* nn_values,
                                  const int32_t* vl_paths, const int32_t* vl_lens, float q_penalty, int64_t B,
                                  int64_t total, void* stream) {
    if (B <= 0 || total <= 0) return 0;
    LeafIn L{leaf_idx, leaf_states, legal_moves, num_legal, priors_per_legal, child_q_values, results};
    hipLaunchKernelGGL(k_expand_backprop, dim3((unsigned)B), dim3(64), 0, (hipStream_t)stream, to_tree(tree), L,
                       nn_values, vl_paths, vl_lens, q_penalty, B, total);
    return finish();
}

int64_t hg_mcts_expand_backprop_dense_workspace(int64_t B, int64_t total) {
    return B <= 0 || total <= 0 ? 0 : 4 * (2 * total + 2 * B);
}

int hg_mcts_expand_backprop_dense_ws(const hg_tree* tree, const float* child_q_values, const int32_t* leaf_idx,
                                     const uint8_t* leaf_states, const uint8_t* legal_moves,
                                     const int32_t* num_legal, const float* priors_per_legal, const int32_t* results,
                                     const float* nn_values, const int32_t* vl_paths, const int32_t* vl_lens,
                                     float q_penalty, int64_t B, int64_t total, void* workspace, void* stream) {
    (void)workspace;  // the plan lives in the workgroup's LDS
    return eb_games(tree, child_q_values, leaf_idx, leaf_states, legal_moves, num_legal, priors_per_legal, results,
                    nn_values, vl_paths, vl_lens, q_penalty, B, total, kEbWaves, (hipStream_t)stream);
}

int hg_mcts_select(const hg_tree* tree, const int8_t* game_active, const int32_t* root_nodes, float c_puct, int64_t B,
                   int W, int32_t* leaf_idx, uint8_t* move_paths, int32_t* path_lens, int32_t* vl_paths,
                   int32_t* vl_lens, void* stream) {
    if (B <= 0 || W <= 0) return 0;
    SelectOut O{leaf_idx, move_paths, path_lens, vl_paths, vl_lens};
    hipLaunchKernelGGL(k_select_legacy, dim3((unsigned)B), dim3(64), 0, (hipStream_t)stream, to_tree(tree), game_active,
                       root_nodes, c_puct, B, (int64_t)W * B, O);
    return finish();
}

int hg_mcts_expand(const hg_tree* tree, const int32_t* leaf_idx, const uint8_t* leaf_states, const uint8_t* legal_moves,
                   const int32_t* num_legal, const float* action_probs, const int32_t* results, int64_t B,
                   int64_t total, int8_t* was_expanded, void* stream) {
    if (B <= 0 || total <= 0) return 0;
    LeafIn L{leaf_idx, leaf_states, legal_moves, num_legal, action_probs, nullptr, results};
    hipLaunchKernelGGL(k_expand_legacy, dim3((unsigned)B), dim3(64), 0, (hipStream_t)stream, to_tree(tree), L, B, total,
                       was_expanded);
    return finish();
}

int hg_mcts_backprop(const hg_tree* tree, const int32_t* leaf_idx, const float* nn_values, const int32_t* vl_paths,
                     const int32_t* vl_lens, const int8_t* was_expanded, int64_t B, int64_t total, void* stream) {
    if (B <= 0 || total <= 0) return 0;
    hipLaunchKernelGGL(k_backprop_legacy, dim3((unsigned)B), dim3(64), 0, (hipStream_t)stream, to_tree(tree), leaf_idx,
                       nn_values, vl_paths, vl_lens, was_expanded, B, total);
    return finish();
}

int hg_mcts_expand_backprop(const hg_tree* tree, const int32_t* leaf_idx, const uint8_t* leaf_states,
                            const uint8_t* legal_moves, const int32_t* num_legal, const float* action_probs,
                            const int32_t* results, const float* nn_values, const int32_t* vl_paths,
                            const int32_t* vl_lens, int64_t B, int64_t total, void* stream) {
    if (B <= 0 || total <= 0) return 0;
    LeafIn L{leaf_idx, leaf_states, legal_moves, num_legal, action_probs, nullptr, results};
    hipLaunchKernelGGL(k_expand_backprop_legacy, dim3((unsigned)B), dim3(64), 0, (hipStream_t)stream, to_tree(tree), L,
                       nn_values, vl_paths, vl_lens, B, total);
    return finish();
}

int hg_mcts_extract_policy(const hg_tree* tree, const int32_t* move_numbers, const int32_t* root_nodes,
                           float temperature, int temp_drop_move, float pruning_threshold, int64_t B, float* policies,
                           void* stream) {
    if (B <= 0) return 0;
    hipLaunchKernelGGL(k_extract_policy, dim3((unsigned)B), dim3(64), 0, (hipStream_t)stream, to_tree(tree),
                       move_numbers, root_nodes, temperature, temp_drop_move, pruning_threshold, B, policies);
    return finish();
}

int hg_mcts_root_noise(const hg_tree* tree, const float* noise, const int32_t* root_nodes, int max_children_pad,
                       float dir_eps, float root_policy_temp, int64_t B, void* stream) {
    if (B <= 0) return 0;
    hipLaunchKernelGGL(k_root_noise, dim3((unsigned)((B + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       to_tree(tree), noise, root_nodes, max_children_pad, dir_eps, root_policy_temp, B);
    return finish();
}

int hg_mcts_wave_root_slots(const hg_tree* tree, const uint8_t* root_states, const int8_t* game_active,
                            const int32_t* root_nodes, const int32_t* root_slots, int num_candidates,
                            int max_root_children, float c_puct, int64_t B, int W, int deterministic_non_root,
                            float non_root_sigma, float q_penalty, const hg_fnn_net* net,
                            const hg_wave_buffers* buf, void* stream) {
    if (B <= 0 || W <= 0 || num_candidates <= 0) return 0;
    if (!tree || !net || !buf || net->F != 122) return (int)hipErrorInvalidValue;
    const int64_t T = (int64_t)W * num_candidates * B;
    if (T > buf->capacity || T > (int64_t)INT32_MAX) return (int)hipErrorInvalidValue;
    hipStream_t s = (hipStream_t)stream;
    // the wave's readers of the path rows (replay, expansion + backup) stop at
    // the recorded lengths: the rows' tails are not written
    int e = select_root_slots(tree, game_active, root_nodes, root_slots, num_candidates, max_root_children, c_puct, B,
                              W, deterministic_non_root, non_root_sigma, q_penalty,
                              SelectOut{buf->leaf_idx, buf->move_paths, buf->path_lens, buf->vl_paths, buf->vl_lens, 0},
                              s);
    if (e) return e;
    // replay into the leaf rows (idle simulations: zero rows) with each leaf's
    // result, and the leaves' legal lists + features, in one launch
    hipLaunchKernelGGL(k_replay_legal, dim3((unsigned)((T + kPosPerWave - 1) / kPosPerWave)), dim3(64), 0, s,
                       root_states, B, buf->leaf_states, buf->move_paths, buf->path_lens, buf->leaf_idx, T,
                       buf->results, buf->legal_moves, buf->num_legal, buf->features);
    if ((e = finish())) return e;
    // the leaf evaluation, the search counters (when asked for) in its first launch
    if ((e = hw::leaf_eval_lists(buf->leaf_states, buf->legal_moves, buf->num_legal, buf->features, T, net->F,
                                 net->fc1_w, net->fc1_b, net->ln_w, net->ln_b, net->fc2_w, net->fc2_b,
                                 net->value_w, net->value_b, net->action1_w, net->action1_b, net->action2_w,
                                 net->action2_b, buf->leaf_workspace, buf->priors, buf->values, buf->child_q,
                                 buf->leaf_idx, buf->vl_lens, buf->stats, s, false)))
        return e;
    return eb_games(tree, buf->child_q, buf->leaf_idx, buf->leaf_states, buf->legal_moves, buf->num_legal,
                    buf->priors, buf->results, buf->values, buf->vl_paths, buf->vl_lens, q_penalty, B, T,
                    num_candidates, s);
}

int hg_gumbel_halving(const hg_tree* tree, const int32_t* root_nodes, const int32_t* candidates, int C,
                      const float* base, float c_visit, float c_scale, int root_q_min_visits, int keep, int64_t B,
                      int32_t* cand_out, int64_t* chosen, void* stream) {
    if (B <= 0) return 0;
    if (!tree || C < 1 || C > 64 || keep < 0 || keep > C) return (int)hipErrorInvalidValue;
    if ((keep > 0 && !cand_out) || (keep == 0 && !chosen)) return (int)hipErrorInvalidValue;
    int Cp = 1;
    while (Cp < C) Cp <<= 1;
    const int64_t per = kHalvThreads / Cp;
    hipLaunchKernelGGL(k_gumbel_halving, dim3((unsigned)((B + per - 1) / per)), dim3(kHalvThreads), 0,
                       (hipStream_t)stream, to_tree(tree), root_nodes, candidates, C, Cp, base, c_visit, c_scale,
                       root_q_min_visits, keep, B, cand_out, chosen);
    return finish();
}

int hg_mcts_reset_trees(const hg_tree* tree, const int8_t* reset, int32_t* root_node, int64_t B, void* stream) {
    if (B <= 0) return 0;
    if (B > 65535) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_reset_nodes, dim3(64, (unsigned)B), dim3(256), 0, (hipStream_t)stream, to_tree(tree), reset,
                       B);
    hipLaunchKernelGGL(k_reset_counts, dim3((unsigned)((B + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       tree->node_count, root_node, reset, B);
    return finish();
}

}  // extern "C"
