// hive_leaf.hpp -- the successor-row plan shared by the engine's successor-row
// entry point (hive_engine.hip) and the fused leaf evaluation (hive_fnn.hip),
// and the internal launches the leaf evaluation and the simulation wave
// (hive_mcts.hip) call across files.
//
// The plan of a batch of T leaves with legal counts n[t] (clamped to
// [0, 256]): offsets[t] = n[0] + ... + n[t - 1], total = the sum, and per row
// r < total its leaf a2r[r] and legal slot mi[r] (the rows of leaf t are
// offsets[t] .. offsets[t] + n[t] - 1, in slot order).  The counts stay on
// the device: nothing here synchronises with the host.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hive_wave.hpp"

namespace hw {

// batches of at most kPlanLeaves leaves are planned in one launch of
// 256-thread blocks (rows_plan_block); larger ones in two (offsets, then map)
constexpr int64_t kPlanLeaves = 32768;
__device__ __forceinline__ int clamp_legal(int n) { return n < 0 ? 0 : (n > kMaxLegal ? kMaxLegal : n); }

// Block b of the one-launch plan (256 threads) owns leaves [256 b, 256 b +
// 256): it adds up the clamped counts before its range itself (at most
// kPlanLeaves reads from L2, four counts per load when the counts are 16-byte
// aligned), scans its own counts and writes their offsets; then each wave
// writes its leaves' rows (stores only: no wave waits on another's).
// Sums stay below kPlanLeaves * 256 (int).
__device__ __forceinline__ int clamp4_sum(int4 v) {
    return clamp_legal(v.x) + clamp_legal(v.y) + clamp_legal(v.z) + clamp_legal(v.w);
}
__device__ __forceinline__ void rows_plan_block(const int32_t* __restrict__ nlegal, int64_t T,
                                                int64_t* __restrict__ offsets, int64_t* __restrict__ total,
                                                int64_t* __restrict__ a2r, int64_t* __restrict__ mi, int b) {
    __shared__ int carry_w[4], tot_w[4];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int lo = b * 256;  // a multiple of 4: leaves [0, lo) are whole int4s
    int before = 0;
    if (((uintptr_t)nlegal & 15) == 0) {
        const int4* n4 = reinterpret_cast<const int4*>(nlegal);
#pragma unroll 8
        for (int q = tid; q < lo / 4; q += 256) before += clamp4_sum(n4[q]);
    } else {
#pragma unroll 8
        for (int t = tid; t < lo; t += 256) before += clamp_legal(nlegal[t]);
    }
    const int t = lo + tid;
    const int v = t < T ? clamp_legal(nlegal[t]) : 0;
    const int incl = wave_incl_scan(v);
    const int cw = wave_sum(before);
    if (lane == 0) carry_w[w] = cw;
    if (lane == 63) tot_w[w] = incl;
    __syncthreads();
    int off = carry_w[0] + carry_w[1] + carry_w[2] + carry_w[3] + incl - v;
    for (int k = 0; k < w; k++) off += tot_w[k];
    if (t < T) offsets[t] = off;
    if (tid == 255 && lo + 256 >= T) *total = (int64_t)off + v;  // the block holding leaf T - 1
    // each wave writes its 64 leaves' rows one leaf at a time, the lanes over
    // the leaf's slots (stores of consecutive rows, not one row per lane of
    // 64 different leaves)
    for (int k = 0; k < 64; k++) {
        const int vk = __builtin_amdgcn_readlane(v, k), ok = __builtin_amdgcn_readlane(off, k);
        const int64_t tk = (int64_t)lo + 64 * w + k;
        for (int m = lane; m < vk; m += 64) {
            a2r[ok + m] = tk;
            mi[ok + m] = m;
        }
    }
}

// The successor-row workspace (hg_successor_rows_workspace(T) bytes):
// offsets [T], total [1], a2r [T * 256], mi [T * 256], all int64.
struct RowsPlan {
    int64_t *offsets, *total, *a2r, *mi;
};
inline RowsPlan rows_plan_of(void* workspace, int64_t T) {
    int64_t* o = reinterpret_cast<int64_t*>(workspace);
    return RowsPlan{o, o + T, o + T + 1, o + T + 1 + T * kMaxLegal};
}

// hive_engine.hip: the plan of more than kPlanLeaves leaves (offsets, then the
// row map), and the successor features of the planned rows
int successor_rows_plan_large(const int32_t* num_legal, int64_t T, void* workspace, hipStream_t s);
int successor_rows_after_plan(const uint8_t* states, const uint8_t* legal_moves, int64_t T, void* workspace,
                              float* features, hipStream_t s);

// hive_fnn.hip: hg_fnn_leaf_eval_lists, and with `stats` (int64[4]) the
// simulation wave's search counters of hg_mcts_wave_stats over leaf_idx,
// num_legal and vl_lens added in its first launch; without `dense` the
// priors / child-Q rows are written up to each leaf's legal count only (the
// simulation wave's expansion reads no further)
int leaf_eval_lists(const uint8_t* leaf_states, const uint8_t* legal_moves, const int32_t* num_legal,
                    const float* root_features, int64_t T, int F, const float* fc1_w, const float* fc1_b,
                    const float* ln_w, const float* ln_b, const float* fc2_w, const float* fc2_b,
                    const float* value_w, float value_b, const float* action1_w, const float* action1_b,
                    const float* action2_w, float action2_b, void* workspace, float* priors, float* root_values,
                    float* child_q, const int32_t* leaf_idx, const int32_t* vl_lens, int64_t* stats,
                    hipStream_t stream, bool dense = true);

}  // namespace hw
