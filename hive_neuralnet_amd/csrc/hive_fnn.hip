// hive_fnn.hip -- the FNN leaf evaluation of the self-play search, fused.
//
// The reference evaluates a batch of leaves with a chain of torch ops
// (fnn_mcts_orchestrator.py:243-316 over fnn_network.py:175-220): legal-slot
// masks, row lists, successor features, concatenation, fc1, sigmoid,
// LayerNorm, fc2, value head, action tower over [root | successor]
// embeddings, scatter into [T, 256] logits, softmax, child-Q scatter.  Here
// the GEMMs stay with hipBLASLt (torch.addmm) and the rest collapses into
// two kernels:
//
//   k_sigmoid_layernorm  h <- LayerNorm(sigmoid(h)) in place, per 64-wide row
//                        (fnn_network.py:175-187, eps 1e-5, biased variance);
//   k_leaf_heads         per leaf: child values tanh(e_succ . wv + bv), action
//                        logits a2 . sigmoid(S_succ + R_root) + b2 (the action
//                        tower's first layer split into its successor half S
//                        and root half R, fnn_network.py:204-220), softmax
//                        over the leaf's legal slots, priors / child Q
//                        (= -child value) written as [T, 256] rows with zero
//                        padding, and the leaf's own value.
//
// Floating point: fp32 throughout with the same operations as the torch
// path; summation orders differ (GEMM split, reductions), so results agree
// with the torch path to ~1e-6 relative, not bit for bit.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hive_gpu.h"

namespace {

constexpr int kE = 64;  // embedding / hidden width of the FNN presets this kernel serves
constexpr int kSlots = 256;

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
__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

// one 64-lane wave per row, lane = column
__global__ __launch_bounds__(256) void k_sigmoid_layernorm(float* __restrict__ h, const float* __restrict__ gamma,
                                                           const float* __restrict__ beta, int64_t rows) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    float* x = h + row * kE;
    float v = sigmoidf_(x[lane]);
    float mean = wave_sum_f(v) / (float)kE;
    float d = v - mean;
    float var = wave_sum_f(d * d) / (float)kE;
    x[lane] = d / sqrtf(var + 1e-5f) * gamma[lane] + beta[lane];
}

// One wave per leaf t.  E: [T + N, 64] embeddings (leaf rows 0..T-1, successor
// rows T..T+N-1); S: [N, 64] successor halves of the action tower's first
// layer (no bias); R: [T, 64] root halves with the bias; offsets[t] = first
// successor row of leaf t, n[t] its legal-slot count.
__global__ __launch_bounds__(256) void k_leaf_heads(const float* __restrict__ E, const float* __restrict__ S,
                                                    const float* __restrict__ R, const int64_t* __restrict__ offsets,
                                                    const int32_t* __restrict__ nlegal, int64_t T,
                                                    const float* __restrict__ wv, float bv,
                                                    const float* __restrict__ wa2, float ba2,
                                                    float* __restrict__ priors, float* __restrict__ root_values,
                                                    float* __restrict__ child_q) {
    __shared__ float sR[4][kE], sWv[kE], sWa[kE];
    const int lane = threadIdx.x & 63, wv_i = threadIdx.x >> 6;
    const int64_t t = (int64_t)blockIdx.x * 4 + wv_i;
    if (threadIdx.x < kE) {
        sWv[threadIdx.x] = wv[threadIdx.x];
        sWa[threadIdx.x] = wa2[threadIdx.x];
    }
    if (t < T) sR[wv_i][lane] = R[t * kE + lane];
    __syncthreads();
    if (t >= T) return;
    // the leaf's own value
    float rv = wave_sum_f(E[t * kE + lane] * sWv[lane]);
    if (lane == 0) root_values[t] = tanhf(rv + bv);
    int n = nlegal[t];
    n = n < 0 ? 0 : (n > kSlots ? kSlots : n);
    const int64_t base = offsets[t];
    // lane i handles slots i, i + 64, ...: child value and action logit
    float logit[4], cv[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        int i = lane + 64 * k;
        logit[k] = -INFINITY;
        cv[k] = 0.0f;
        if (i < n) {
            const float4* e4 = reinterpret_cast<const float4*>(E + (T + base + i) * kE);
            const float4* s4 = reinterpret_cast<const float4*>(S + (base + i) * kE);
            float v = 0.0f, a = 0.0f;
#pragma unroll
            for (int j = 0; j < kE / 4; j++) {
                float4 e = e4[j], s = s4[j];
                v += e.x * sWv[4 * j] + e.y * sWv[4 * j + 1] + e.z * sWv[4 * j + 2] + e.w * sWv[4 * j + 3];
                a += sigmoidf_(s.x + sR[wv_i][4 * j]) * sWa[4 * j] + sigmoidf_(s.y + sR[wv_i][4 * j + 1]) * sWa[4 * j + 1] +
                     sigmoidf_(s.z + sR[wv_i][4 * j + 2]) * sWa[4 * j + 2] +
                     sigmoidf_(s.w + sR[wv_i][4 * j + 3]) * sWa[4 * j + 3];
            }
            cv[k] = tanhf(v + bv);
            logit[k] = a + ba2;
        }
    }
    float m = fmaxf(fmaxf(logit[0], logit[1]), fmaxf(logit[2], logit[3]));
    m = wave_max_f(m);
    float ex[4], s = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        int i = lane + 64 * k;
        ex[k] = i < n ? expf(logit[k] - m) : 0.0f;
        s += ex[k];
    }
    s = wave_sum_f(s);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        int i = lane + 64 * k;
        priors[t * kSlots + i] = i < n ? ex[k] / s : 0.0f;
        child_q[t * kSlots + i] = i < n ? -cv[k] : 0.0f;
    }
}

inline int grid_for(int64_t n, int per) { return (int)((n + per - 1) / per); }

}  // namespace

extern "C" {

int hg_fnn_sigmoid_layernorm(float* h, const float* gamma, const float* beta, int64_t rows, void* stream) {
    if (rows <= 0) return 0;
    hipLaunchKernelGGL(k_sigmoid_layernorm, dim3(grid_for(rows, 4)), dim3(256), 0, (hipStream_t)stream, h, gamma,
                       beta, rows);
    return (int)hipGetLastError();
}

int hg_fnn_leaf_heads(const float* emb, const float* succ_half, const float* root_half, const int64_t* offsets,
                      const int32_t* num_legal, int64_t T, const float* value_w, float value_b, const float* action_w,
                      float action_b, float* priors, float* root_values, float* child_q, void* stream) {
    if (T <= 0) return 0;
    hipLaunchKernelGGL(k_leaf_heads, dim3(grid_for(T, 4)), dim3(256), 0, (hipStream_t)stream, emb, succ_half,
                       root_half, offsets, num_legal, T, value_w, value_b, action_w, action_b, priors, root_values,
                       child_q);
    return (int)hipGetLastError();
}

}  // extern "C"
