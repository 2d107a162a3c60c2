// hive_fnn.hip -- the FNN leaf evaluation of the self-play search, fused.
//
// The reference evaluates a batch of leaves with a chain of torch ops
// (fnn_mcts_orchestrator.py:243-316 over fnn_network.py:175-220): legal-slot
// masks, row lists, successor features, concatenation, fc1, sigmoid,
// LayerNorm, fc2, value head, action tower over [root | successor]
// embeddings, scatter into [T, 256] logits, softmax, child-Q scatter.  Here
// the whole network runs in one kernel per row kind, with the weights held in
// LDS and the three layer products on fp32 matrix cores:
//
//   k_leaf_mlp<root>   per leaf row: embedding e = fc2(LN(sigmoid(fc1 x))),
//                      value tanh(value_fc e), and the root half of the
//                      action tower's first layer r = Wr e + b (Wr =
//                      action_fc1.weight[:, :64]), kept as [T][64];
//   k_leaf_mlp<succ>   per successor row: e as above, child value
//                      tanh(value_fc e), and the action logit
//                      action_fc2(sigmoid(Ws e + r[leaf])) (Ws =
//                      action_fc1.weight[:, 64:]), so [root | successor] is
//                      never materialised;
//   k_leaf_softmax     per leaf: softmax of its logits over its legal slots,
//                      priors / child Q (= -child value) as [T][256] rows,
//                      zero beyond the legal count.
//
// Matrix-core layout (v_mfma_f32_16x16x4f32, D = A.B + C, A 16x4, B 4x16):
// lane l holds A[l%16][l/16], B[l/16][l%16] and D[4(l/16)+i][l%16] in its
// four accumulator registers i.  A wave evaluates 16 rows at a time and
// computes every layer transposed, out^T = W . in^T: A = 16 output units of
// W, B = the inputs of the 16 rows, so after a layer lane l holds, for row
// l%16, the 16 units {16t + 4(l/16) + i : t, i < 4} of its output.  Those are
// exactly the B operands the next layer needs when the K index of step s for
// lane group g = l/16 is 16(s/4) + 4g + s%4: no transposes, no LDS traffic
// between layers.  The weights are stored in LDS pre-permuted to that K
// order ([step][lane][tile] float4 per lane, conflict-free 16-byte reads).
// The first layer reads the features in their natural order, K index 32g + s
// for lane group g (a lane loads 32 consecutive features of its row).
//
// LayerNorm, value and logit reductions over the 64 units of a row are a
// sum over the lane's 16 units plus two cross-lane steps (lanes l, l^16,
// l^32, l^48 share a row).
//
// Floating point: fp32 throughout with the reference's operations (eps 1e-5,
// biased variance; sigmoid from the hardware exp2 / reciprocal);
// summation orders differ from torch's GEMMs, so results agree with the
// torch composition to ~1e-6 relative, not bit for bit.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hive_gpu.h"
#include "hive_leaf.hpp"

namespace {

constexpr int kE = 64;       // hidden / embedding / action-tower width served here
constexpr int kFMax = 128;   // feature rows up to 128 wide (Hive FNN: 122)
constexpr int kSlots = 256;  // legal-slot rows of priors / child Q
// 8 waves share one LDS copy of the weights: 2 resident blocks (67 KB LDS
// each) per CU give 4 waves per SIMD to overlap the element-wise work and
// loads with the matrix cores
constexpr int kBlockWaves = 8;
constexpr int kMaxBlocks = 512;  // 2 resident blocks on each of 256 CUs

typedef float f4 __attribute__((ext_vector_type(4)));

struct MlpLds {
    f4 w1[32][64];  // fc1, step s = K index 32g + s
    f4 w2[16][64];  // fc2, step s = K index 16(s/4) + 4g + s%4
    f4 w3[16][64];  // action_fc1 root half (root rows) or successor half (successor rows)
    float vec[7][kE];
};
enum { kB1, kLnW, kLnB, kB2, kWv, kWa2, kBa1 };

// The network laid out once per evaluation in the order the MLP kernels keep
// in LDS (pack_net_at, in the evaluation's first launch), so that each of
// their blocks fills LDS with straight 16-byte copies instead of gathering
// and permuting the weights itself.
struct PackedNet {
    f4 w1[32][64];
    f4 w2[16][64];
    f4 w3[2][16][64];  // action_fc1: root half, successor half
    float vec[7][kE];
};

// element i of a [step][lane][tile] array: unit m = 16 tile + lane % 16 and the
// step / lane group dependent K index (fc1: 32 g + s; the 64-wide layers:
// 16 (s / 4) + 4 g + s % 4)
__device__ __forceinline__ void perm_index(int i, bool first, int& m, int& k) {
    const int t = i & 3, l = (i >> 2) & 63, s = i >> 8;
    m = 16 * t + (l & 15);
    k = first ? 32 * (l >> 4) + s : 16 * (s >> 2) + 4 * (l >> 4) + (s & 3);
}

// thread i of the packing writes float i of the packed layout (k_leaf_prep's
// packing blocks)
__device__ __forceinline__ void pack_net_at(int i, const float* __restrict__ w1, int F, const float* __restrict__ b1,
                                            const float* __restrict__ lnw, const float* __restrict__ lnb,
                                            const float* __restrict__ w2, const float* __restrict__ b2,
                                            const float* __restrict__ wv, const float* __restrict__ a1w,
                                            const float* __restrict__ a1b, const float* __restrict__ a2w,
                                            PackedNet* __restrict__ out) {
    constexpr int n1 = 32 * 64 * 4, n2 = 16 * 64 * 4;
    int m, k;
    if (i < n1) {
        perm_index(i, true, m, k);
        reinterpret_cast<float*>(&out->w1[0][0])[i] = k < F ? w1[m * F + k] : 0.0f;
    } else if (i < n1 + n2) {
        perm_index(i - n1, false, m, k);
        reinterpret_cast<float*>(&out->w2[0][0])[i - n1] = w2[m * kE + k];
    } else if (i < n1 + 3 * n2) {
        const int j = i - n1 - n2, half = j / n2;
        perm_index(j - half * n2, false, m, k);
        reinterpret_cast<float*>(&out->w3[0][0][0])[j] = a1w[m * 2 * kE + half * kE + k];
    } else if (i < n1 + 3 * n2 + kE) {
        const int u = i - n1 - 3 * n2;
        out->vec[kB1][u] = b1[u];
        out->vec[kLnW][u] = lnw[u];
        out->vec[kLnB][u] = lnb[u];
        out->vec[kB2][u] = b2[u];
        out->vec[kWv][u] = wv[u];
        out->vec[kWa2][u] = a2w[u];
        out->vec[kBa1][u] = a1b[u];
    }
}
constexpr int kPackThreads = 32 * 64 * 4 + 3 * 16 * 64 * 4 + kE;
constexpr int kPackBlocks = (kPackThreads + 255) / 256;

// The first launch of a fused leaf evaluation, three kinds of 256-thread
// blocks side by side (none waits for another): the successor-row plan of
// up to kPlanLeaves leaves (plan_blocks blocks, hw::rows_plan_block), the
// network in the MLP kernels' layout (kPackBlocks blocks, pack_net_at)
// and, with `stats`, the simulation wave's search counters (one block per
// 1,024 simulations: leaves reached, their legal counts, their virtual-loss
// lengths, rows; integer sums added with device atomics).
__global__ __launch_bounds__(256) void k_leaf_prep(const int32_t* __restrict__ nlegal, int64_t T, int plan_blocks,
                                                   hw::RowsPlan plan, const float* __restrict__ w1, int F,
                                                   const float* __restrict__ b1, const float* __restrict__ lnw,
                                                   const float* __restrict__ lnb, const float* __restrict__ w2,
                                                   const float* __restrict__ b2, const float* __restrict__ wv,
                                                   const float* __restrict__ a1w, const float* __restrict__ a1b,
                                                   const float* __restrict__ a2w, PackedNet* __restrict__ pk,
                                                   const int32_t* __restrict__ leaf_idx,
                                                   const int32_t* __restrict__ vl_lens,
                                                   unsigned long long* __restrict__ stats) {
    int b = (int)blockIdx.x;
    if (b < plan_blocks) {
        hw::rows_plan_block(nlegal, T, plan.offsets, plan.total, plan.a2r, plan.mi, b);
        return;
    }
    b -= plan_blocks;
    if (b < kPackBlocks) {
        pack_net_at(b * 256 + (int)threadIdx.x, w1, F, b1, lnw, lnb, w2, b2, wv, a1w, a1b, a2w, pk);
        return;
    }
    b -= kPackBlocks;
    __shared__ unsigned long long part[3][4];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    unsigned long long a = 0, n = 0, d = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int64_t i = (int64_t)b * 1024 + k * 256 + tid;
        if (i < T && leaf_idx[i] >= 0) {
            a += 1;
            n += (unsigned long long)(long long)nlegal[i];
            d += (unsigned long long)(long long)vl_lens[i];
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        a += __shfl_xor(a, off);
        n += __shfl_xor(n, off);
        d += __shfl_xor(d, off);
    }
    if (lane == 0) {
        part[0][w] = a;
        part[1][w] = n;
        part[2][w] = d;
    }
    __syncthreads();
    if (tid < 3) {
        atomicAdd(&stats[tid], part[tid][0] + part[tid][1] + part[tid][2] + part[tid][3]);
    } else if (tid == 3 && b == 0) {
        atomicAdd(&stats[3], (unsigned long long)T);
    }
}

// sigmoid from the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32):
// ~1e-6 relative against the correctly rounded form, inside the 1e-5
// tolerance the network's outputs are held to, at a fraction of expf's and
// the IEEE division's instructions (128 sigmoids per successor row)
__device__ __forceinline__ float sigmoidf_(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504088896341f));
}

// sum over the four lanes l, l^16, l^32, l^48 (one row)
__device__ __forceinline__ float row_sum(float v) {
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

__device__ __forceinline__ f4 mfma(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f4 vec4(const MlpLds& L, int which, int t, int g) {
    return *reinterpret_cast<const f4*>(&L.vec[which][16 * t + 4 * g]);
}

// X: [rows][F] features (F even, <= 128, 8-byte aligned rows).
// kRoot: R[rows][64] <- Wr e + b_a1, value[rows] <- tanh(wv . e + bv).
// !kRoot: row -> leaf = succ_leaf[row]; value[rows] <- tanh(wv . e + bv),
//         logit[rows] <- wa2 . sigmoid(Ws e + R[leaf]) + ba2.
template <bool kRoot>
__global__ __launch_bounds__(64 * kBlockWaves) void k_leaf_mlp(const float* __restrict__ X, int64_t rows, int F,
                                                  const int64_t* __restrict__ succ_leaf, int64_t T,
                                                  const float* __restrict__ w1, const float* __restrict__ b1,
                                                  const float* __restrict__ lnw, const float* __restrict__ lnb,
                                                  const float* __restrict__ w2, const float* __restrict__ b2,
                                                  const float* __restrict__ wv, float bv, const float* __restrict__ a1w,
                                                  const float* __restrict__ a1b, const float* __restrict__ a2w, float ba2,
                                                  float* __restrict__ R, float* __restrict__ value,
                                                  float* __restrict__ logit, const int64_t* __restrict__ rows_dev,
                                                  const PackedNet* __restrict__ pk) {
    __shared__ MlpLds L;
    if (rows_dev) rows = *rows_dev;  // row count held on the device
    const int64_t ntiles = (rows + 15) >> 4;
    // 16-row tiles dealt over the blocks first (tile = block + grid * (wave +
    // kBlockWaves * round)): a short batch spreads over all CUs, and a block
    // with no tile leaves before filling LDS
    if ((int64_t)blockIdx.x >= ntiles) return;
    if (pk) {  // the packed layout: straight 16-byte copies, every load issued before the first store
        constexpr int kT = 64 * kBlockWaves, k12 = 48 * 64 / kT, k3 = 16 * 64 / kT;
        static_assert(48 * 64 % kT == 0 && 16 * 64 % kT == 0 && 7 * kE / 4 <= kT, "whole copy rounds");
        const int tid = threadIdx.x;
        const f4* src = &pk->w1[0][0];
        const f4* s3 = &pk->w3[kRoot ? 0 : 1][0][0];
        f4 c12[k12], c3[k3], cv = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < k12; k++) c12[k] = src[tid + k * kT];  // w1, w2
#pragma unroll
        for (int k = 0; k < k3; k++) c3[k] = s3[tid + k * kT];
        if (tid < 7 * kE / 4) cv = reinterpret_cast<const f4*>(&pk->vec[0][0])[tid];
        f4* dst = &L.w1[0][0];
#pragma unroll
        for (int k = 0; k < k12; k++) dst[tid + k * kT] = c12[k];
#pragma unroll
        for (int k = 0; k < k3; k++) (&L.w3[0][0])[tid + k * kT] = c3[k];
        if (tid < 7 * kE / 4) reinterpret_cast<f4*>(&L.vec[0][0])[tid] = cv;
    } else {  // permuted weights gathered into LDS (perm_index)
        int m, k;
        float* l1 = reinterpret_cast<float*>(&L.w1[0][0]);
        for (int i = threadIdx.x; i < 32 * 64 * 4; i += blockDim.x) {
            perm_index(i, true, m, k);
            l1[i] = k < F ? w1[m * F + k] : 0.0f;
        }
        float* l2 = reinterpret_cast<float*>(&L.w2[0][0]);
        float* l3 = reinterpret_cast<float*>(&L.w3[0][0]);
        for (int i = threadIdx.x; i < 16 * 64 * 4; i += blockDim.x) {
            perm_index(i, false, m, k);
            l2[i] = w2[m * kE + k];
            l3[i] = a1w[m * 2 * kE + (kRoot ? 0 : kE) + k];
        }
        if (threadIdx.x < kE) {
            const int u = threadIdx.x;
            L.vec[kB1][u] = b1[u];
            L.vec[kLnW][u] = lnw[u];
            L.vec[kLnB][u] = lnb[u];
            L.vec[kB2][u] = b2[u];
            L.vec[kWv][u] = wv[u];
            L.vec[kWa2][u] = a2w[u];
            L.vec[kBa1][u] = a1b[u];
        }
    }
    __syncthreads();

    const int lane = threadIdx.x & 63, g = lane >> 4;
    for (int64_t tile = (int64_t)blockIdx.x + (int64_t)gridDim.x * (threadIdx.x >> 6); tile < ntiles;
         tile += (int64_t)gridDim.x * kBlockWaves) {
        // the weights are re-read from LDS in every tile: hoisted out of the
        // loop they would take ~400 registers and leave one wave per SIMD
        __asm__ volatile("" ::: "memory");
        const int64_t row = tile * 16 + (lane & 15);
        const bool ok = row < rows;
        // successor rows: the leaf's root half of the action tower, fetched first
        f4 rh[4];
        if constexpr (!kRoot) {
            int64_t leaf = ok ? succ_leaf[row] : 0;
            leaf = leaf < 0 ? 0 : (leaf >= T ? T - 1 : leaf);
#pragma unroll
            for (int t = 0; t < 4; t++) rh[t] = *reinterpret_cast<const f4*>(R + leaf * kE + 16 * t + 4 * g);
        }
        // features 32g .. 32g+31 of this lane's row
        float x[32];
        const float* xr = X + (ok ? row : 0) * F + 32 * g;
#pragma unroll
        for (int p = 0; p < 16; p++) {
            float2 v = make_float2(0.0f, 0.0f);
            if (ok && 32 * g + 2 * p < F) v = *reinterpret_cast<const float2*>(xr + 2 * p);
            x[2 * p] = v.x;
            x[2 * p + 1] = v.y;
        }
        // fc1
        f4 acc[4];
#pragma unroll
        for (int t = 0; t < 4; t++) acc[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 32; s++) {
            const f4 a = L.w1[s][lane];
            acc[0] = mfma(a.x, x[s], acc[0]);
            acc[1] = mfma(a.y, x[s], acc[1]);
            acc[2] = mfma(a.z, x[s], acc[2]);
            acc[3] = mfma(a.w, x[s], acc[3]);
        }
        // sigmoid + LayerNorm over the row's 64 units
        float sum = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const f4 b = vec4(L, kB1, t, g);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                acc[t][i] = sigmoidf_(acc[t][i] + b[i]);
                sum += acc[t][i];
            }
        }
        const float mean = row_sum(sum) / (float)kE;
        float sq = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                acc[t][i] -= mean;
                sq += acc[t][i] * acc[t][i];
            }
        const float rstd = 1.0f / sqrtf(row_sum(sq) / (float)kE + 1e-5f);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const f4 w = vec4(L, kLnW, t, g), b = vec4(L, kLnB, t, g);
#pragma unroll
            for (int i = 0; i < 4; i++) acc[t][i] = acc[t][i] * rstd * w[i] + b[i];
        }
        // fc2 -> embedding
        f4 e[4];
#pragma unroll
        for (int t = 0; t < 4; t++) e[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 16; s++) {
            const f4 a = L.w2[s][lane];
            const float b = acc[s >> 2][s & 3];
            e[0] = mfma(a.x, b, e[0]);
            e[1] = mfma(a.y, b, e[1]);
            e[2] = mfma(a.z, b, e[2]);
            e[3] = mfma(a.w, b, e[3]);
        }
        float v = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const f4 b = vec4(L, kB2, t, g), w = vec4(L, kWv, t, g);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                e[t][i] += b[i];
                v += e[t][i] * w[i];
            }
        }
        v = tanhf(row_sum(v) + bv);
        // action tower, first layer (root or successor half)
        f4 h[4];
#pragma unroll
        for (int t = 0; t < 4; t++) h[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 16; s++) {
            const f4 a = L.w3[s][lane];
            const float b = e[s >> 2][s & 3];
            h[0] = mfma(a.x, b, h[0]);
            h[1] = mfma(a.y, b, h[1]);
            h[2] = mfma(a.z, b, h[2]);
            h[3] = mfma(a.w, b, h[3]);
        }
        if constexpr (kRoot) {
            if (ok) {
#pragma unroll
                for (int t = 0; t < 4; t++)
                    *reinterpret_cast<f4*>(R + row * kE + 16 * t + 4 * g) = h[t] + vec4(L, kBa1, t, g);
                if (g == 0) value[row] = v;
            }
        } else {
            float a = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const f4 w = vec4(L, kWa2, t, g);
#pragma unroll
                for (int i = 0; i < 4; i++) a += sigmoidf_(h[t][i] + rh[t][i]) * w[i];
            }
            a = row_sum(a) + ba2;
            if (ok && g == 0) {
                value[row] = v;
                logit[row] = a;
            }
        }
    }
}

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// One wave per leaf t: softmax of logit[offsets[t] .. + n) into priors[t],
// child_q[t][i] = -child value; zero beyond n.
__global__ __launch_bounds__(256) void k_leaf_softmax(const float* __restrict__ logit, const float* __restrict__ cval,
                                                      const int64_t* __restrict__ offsets,
                                                      const int32_t* __restrict__ nlegal, int64_t T,
                                                      float* __restrict__ priors, float* __restrict__ child_q,
                                                      int dense) {
    const int lane = threadIdx.x & 63;
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    int n = nlegal[t];
    n = n < 0 ? 0 : (n > kSlots ? kSlots : n);
    const int64_t base = offsets[t];
    float lg[4], cv[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int i = lane + 64 * k;
        lg[k] = i < n ? logit[base + i] : -INFINITY;
        cv[k] = i < n ? cval[base + i] : 0.0f;
    }
    const float m = wave_max_f(fmaxf(fmaxf(lg[0], lg[1]), fmaxf(lg[2], lg[3])));
    float ex[4], s = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        ex[k] = lane + 64 * k < n ? expf(lg[k] - m) : 0.0f;
        s += ex[k];
    }
    s = wave_sum_f(s);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int i = lane + 64 * k;
        if (i < n || dense) {  // `dense`: the rows' tails zeroed, else left as they are
            priors[t * kSlots + i] = i < n ? ex[k] / s : 0.0f;
            child_q[t * kSlots + i] = i < n ? -cv[k] : 0.0f;
        }
    }
}

inline int grid_for(int64_t n, int per) { return (int)((n + per - 1) / per); }
// one block per 16-row tile up to kMaxBlocks (the kernels deal tiles over the
// blocks first, so a short batch runs one tile per CU)
inline int mlp_blocks(int64_t rows) {
    const int64_t b = (rows + 15) / 16;
    return (int)(b < kMaxBlocks ? b : kMaxBlocks);
}

}  // namespace

extern "C" {

int hg_fnn_leaf_eval(const float* features, int64_t T, int64_t N, int F, const int64_t* offsets,
                     const int32_t* num_legal, const int64_t* succ_leaf, const float* fc1_w, const float* fc1_b,
                     const float* ln_w, const float* ln_b, const float* fc2_w, const float* fc2_b,
                     const float* value_w, float value_b, const float* action1_w, const float* action1_b,
                     const float* action2_w, float action2_b, float* workspace, float* priors, float* root_values,
                     float* child_q, void* stream) {
    if (T < 0 || N < 0 || F <= 0 || F > kFMax || (F & 1)) return (int)hipErrorInvalidValue;
    if (((uintptr_t)features & 7) || ((uintptr_t)workspace & 15)) return (int)hipErrorInvalidValue;
    if (T == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    float* R = workspace;           // [T][64]
    float* logit = R + T * kE;      // [N]
    float* cval = logit + N;        // [N]
    hipLaunchKernelGGL(k_leaf_mlp<true>, dim3(mlp_blocks(T)), dim3(64 * kBlockWaves), 0, st, features, T, F,
                       nullptr, T, fc1_w, fc1_b, ln_w, ln_b, fc2_w, fc2_b, value_w, value_b, action1_w, action1_b,
                       action2_w, action2_b, R, root_values, nullptr, nullptr, nullptr);
    if (N > 0)
        hipLaunchKernelGGL(k_leaf_mlp<false>, dim3(mlp_blocks(N)), dim3(64 * kBlockWaves), 0, st, features + T * F,
                           N, F, succ_leaf, T, fc1_w, fc1_b, ln_w, ln_b, fc2_w, fc2_b, value_w, value_b, action1_w,
                           action1_b, action2_w, action2_b, R, cval, logit, nullptr, nullptr);
    hipLaunchKernelGGL(k_leaf_softmax, dim3(grid_for(T, 4)), dim3(256), 0, st, logit, cval, offsets, num_legal, T,
                       priors, child_q, 1);
    return (int)hipGetLastError();
}

int64_t hg_fnn_leaf_eval_lists_workspace(int64_t T, int F) {
    if (T <= 0) return 0;
    const int64_t cap = T * kSlots;
    int64_t b = hg_successor_rows_workspace(T);           // offsets, total, row map
    b = (b + 255) & ~(int64_t)255;
    b += cap * F * (int64_t)sizeof(float);                // successor features
    b = (b + 255) & ~(int64_t)255;
    b += (T * kE + 2 * cap) * (int64_t)sizeof(float);     // root half of the action tower, logits, child values
    b = (b + 255) & ~(int64_t)255;
    b += (int64_t)sizeof(PackedNet);                      // the network in the kernels' LDS order
    return b;
}

int hg_fnn_leaf_eval_lists(const uint8_t* leaf_states, const uint8_t* legal_moves, const int32_t* num_legal,
                           const float* root_features, int64_t T, int F, const float* fc1_w, const float* fc1_b,
                           const float* ln_w, const float* ln_b, const float* fc2_w, const float* fc2_b,
                           const float* value_w, float value_b, const float* action1_w, const float* action1_b,
                           const float* action2_w, float action2_b, void* workspace, float* priors,
                           float* root_values, float* child_q, void* stream) {
    return hw::leaf_eval_lists(leaf_states, legal_moves, num_legal, root_features, T, F, fc1_w, fc1_b, ln_w, ln_b,
                               fc2_w, fc2_b, value_w, value_b, action1_w, action1_b, action2_w, action2_b, workspace,
                               priors, root_values, child_q, nullptr, nullptr, nullptr, (hipStream_t)stream);
}

}  // extern "C"

namespace hw {

int leaf_eval_lists(const uint8_t* leaf_states, const uint8_t* legal_moves, const int32_t* num_legal,
                    const float* root_features, int64_t T, int F, const float* fc1_w, const float* fc1_b,
                    const float* ln_w, const float* ln_b, const float* fc2_w, const float* fc2_b,
                    const float* value_w, float value_b, const float* action1_w, const float* action1_b,
                    const float* action2_w, float action2_b, void* workspace, float* priors, float* root_values,
                    float* child_q, const int32_t* leaf_idx, const int32_t* vl_lens, int64_t* stats,
                    hipStream_t st, bool dense) {
    if (T < 0 || F <= 0 || F > kFMax || (F & 1)) return (int)hipErrorInvalidValue;
    if (((uintptr_t)root_features & 7) || ((uintptr_t)workspace & 255)) return (int)hipErrorInvalidValue;
    if (F != 122) return (int)hipErrorInvalidValue;  // the successor rows are the engine's 122 features
    if (stats && (!leaf_idx || !vl_lens)) return (int)hipErrorInvalidValue;
    if (T == 0) return 0;
    const int64_t cap = T * kSlots;
    uint8_t* base = reinterpret_cast<uint8_t*>(workspace);
    int64_t off = hg_successor_rows_workspace(T);
    const RowsPlan plan = rows_plan_of(workspace, T);
    off = (off + 255) & ~(int64_t)255;
    float* X = reinterpret_cast<float*>(base + off);
    off += cap * F * (int64_t)sizeof(float);
    off = (off + 255) & ~(int64_t)255;
    float* R = reinterpret_cast<float*>(base + off);
    float* logit = R + T * kE;
    float* cval = logit + cap;
    off += (T * kE + 2 * cap) * (int64_t)sizeof(float);
    off = (off + 255) & ~(int64_t)255;
    PackedNet* pk = reinterpret_cast<PackedNet*>(base + off);
    // plan, network layout and counters in one launch (the plan of a batch
    // over kPlanLeaves leaves takes its own two launches first)
    int plan_blocks = 0;
    if (T <= kPlanLeaves) {
        plan_blocks = (int)((T + 255) / 256);
    } else {
        int e = successor_rows_plan_large(num_legal, T, workspace, st);
        if (e) return e;
    }
    const int stat_blocks = stats ? (int)((T + 1023) / 1024) : 0;
    hipLaunchKernelGGL(k_leaf_prep, dim3((unsigned)(plan_blocks + kPackBlocks + stat_blocks)), dim3(256), 0, st,
                       num_legal, T, plan_blocks, plan, fc1_w, F, fc1_b, ln_w, ln_b, fc2_w, fc2_b, value_w,
                       action1_w, action1_b, action2_w, pk, leaf_idx, vl_lens,
                       reinterpret_cast<unsigned long long*>(stats));
    int e = successor_rows_after_plan(leaf_states, legal_moves, T, workspace, X, st);
    if (e) return e;
    hipLaunchKernelGGL(k_leaf_mlp<true>, dim3(mlp_blocks(T)), dim3(64 * kBlockWaves), 0, st, root_features, T, F,
                       nullptr, T, fc1_w, fc1_b, ln_w, ln_b, fc2_w, fc2_b, value_w, value_b, action1_w, action1_b,
                       action2_w, action2_b, R, root_values, nullptr, nullptr, pk);
    hipLaunchKernelGGL(k_leaf_mlp<false>, dim3(mlp_blocks(cap)), dim3(64 * kBlockWaves), 0, st, X, cap, F,
                       plan.a2r, T, fc1_w, fc1_b, ln_w, ln_b, fc2_w, fc2_b, value_w, value_b, action1_w, action1_b,
                       action2_w, action2_b, R, cval, logit, plan.total, pk);
    hipLaunchKernelGGL(k_leaf_softmax, dim3(grid_for(T, 4)), dim3(256), 0, st, logit, cval, plan.offsets,
                       num_legal, T, priors, child_q, dense ? 1 : 0);
    return (int)hipGetLastError();
}

}  // namespace hw
