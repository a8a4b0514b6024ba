// Stage2 split reduction and the prologue kernels of a full decode step.
#pragma once
#include "tq4_device.h"

namespace tq4 {

template <typename T> __device__ __forceinline__ T from_float(float x);
template <> __device__ __forceinline__ float from_float<float>(float x) { return x; }
template <> __device__ __forceinline__ __bf16 from_float<__bf16>(float x) { return (__bf16)x; }
template <> __device__ __forceinline__ _Float16 from_float<_Float16>(float x) { return (_Float16)x; }

template <typename T> __device__ __forceinline__ float to_float(T x) { return (float)x; }

// One wave per (q-head, sequence); lane owns dims 2*lane, 2*lane+1.  Pass 1 takes the
// max LSE over the non-empty splits, pass 2 accumulates exp(lse - max)-weighted rows.
template <typename OutT>
__global__ __launch_bounds__(kWave) void stage2_kernel(const float *__restrict__ mid_o,
                                                      const int32_t *__restrict__ seq_lens,
                                                      OutT *__restrict__ out,
                                                      float *__restrict__ lse, int num_q_heads,
                                                      int num_splits) {
    const int h = blockIdx.x;
    const int b = blockIdx.y;
    const int lane = threadIdx.x;
    const int seq_len = seq_lens[b];
    const int split_len = (seq_len + num_splits - 1) / num_splits;
    // splits [0, live) are the non-empty ones: split s is non-empty iff s * len < seq_len
    const int live = split_len > 0 ? min(num_splits, (seq_len + split_len - 1) / split_len) : 0;
    const float *base = mid_o + ((int64_t)b * num_q_heads + h) * num_splits * (kHeadDim + 1);

    float mx = -INFINITY;
    for (int s = lane; s < live; s += kWave)
        mx = fmaxf(mx, base[(int64_t)s * (kHeadDim + 1) + kHeadDim]);
    mx = wave_max(mx);

    float a0 = 0.f, a1 = 0.f, wsum = 0.f;
    for (int s = 0; s < live; ++s) {
        const float *row = base + (int64_t)s * (kHeadDim + 1);
        const float w = expf(row[kHeadDim] - mx);
        a0 += w * row[2 * lane];
        a1 += w * row[2 * lane + 1];
        wsum += w;
    }
    const float inv = 1.f / wsum;
    OutT *o = out + ((int64_t)b * num_q_heads + h) * kHeadDim;
    o[2 * lane] = from_float<OutT>(a0 * inv);
    o[2 * lane + 1] = from_float<OutT>(a1 * inv);
    if (lane == 0)
        lse[(int64_t)b * num_q_heads + h] = mx + logf(wsum);
}

// q_rot[r, n] = sum_k float(query[r, k]) * rot_t[k, n]; 128 threads (one per output
// column) per group of kRotRows rows; the query rows are staged in LDS.
constexpr int kRotRows = 16;
template <typename InT>
__global__ __launch_bounds__(kHeadDim) void rotate_query_kernel(const InT *__restrict__ query,
                                                               const float *__restrict__ rot_t,
                                                               float *__restrict__ q_rot,
                                                               int rows) {
    __shared__ float qs[kRotRows][kHeadDim];
    const int n = threadIdx.x;
    const int r0 = blockIdx.x * kRotRows;
    const int nr = min(kRotRows, rows - r0);
    for (int i = 0; i < nr; ++i)
        qs[i][n] = to_float<InT>(query[(int64_t)(r0 + i) * kHeadDim + n]);
    __syncthreads();
    float acc[kRotRows];
#pragma unroll
    for (int i = 0; i < kRotRows; ++i)
        acc[i] = 0.f;
    for (int k = 0; k < kHeadDim; ++k) {
        const float w = rot_t[k * kHeadDim + n];
#pragma unroll
        for (int i = 0; i < kRotRows; ++i)
            acc[i] += qs[i][k] * w;
    }
    for (int i = 0; i < nr; ++i)
        q_rot[(int64_t)(r0 + i) * kHeadDim + n] = acc[i];
}

__global__ void pair_lut_kernel(const float *__restrict__ cents, float *__restrict__ lut, int n) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t < n * n) {
        lut[2 * t] = cents[t / n];
        lut[2 * t + 1] = cents[t % n];
    }
}

}  // namespace tq4
