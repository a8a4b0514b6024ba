// Stage2 split reduction and the prologue kernels of a full decode step.
#pragma once
#include "tq4_device.h"

namespace tq4 {

template <typename T> __device__ __forceinline__ T from_float(float x);
template <> __device__ __forceinline__ float from_float<float>(float x) { return x; }
template <> __device__ __forceinline__ __bf16 from_float<__bf16>(float x) { return (__bf16)x; }
template <> __device__ __forceinline__ _Float16 from_float<_Float16>(float x) { return (_Float16)x; }

template <typename T> __device__ __forceinline__ float to_float(T x) { return (float)x; }

// One wave per (q-head, sequence); lane owns dims 2*lane, 2*lane+1.  The non-empty splits
// are merged 32 at a time in one pass: lane i reads split i's LSE while every lane reads its
// two dims of all 32 rows (buffer loads at any 4-byte offset: the 516-byte rows are not
// 8-byte aligned), so a wave has its whole share of mid_o in flight at once; then the
// weights exp(lse_s - max) are broadcast lane by lane.  The first chunk's rows are requested
// before the sequence's length arrives (rows past the non-empty splits, never written, are
// replaced by zeros and weight 0), so the length's latency hides under theirs.  A later
// chunk (more than 32 splits) rescales what came before to its own max.
constexpr int kMergeRows = 32;
template <typename OutT>
__global__ __launch_bounds__(kWave) void stage2_kernel(const float *__restrict__ mid_o,
                                                      const int32_t *__restrict__ seq_lens,
                                                      OutT *__restrict__ out,
                                                      float *__restrict__ lse, int num_q_heads,
                                                      int num_splits) {
    const int h = blockIdx.x;
    const int b = blockIdx.y;
    const int lane = threadIdx.x;
    constexpr int kRow = (kHeadDim + 1) * 4;  // bytes per split row
    const __amdgpu_buffer_rsrc_t rows = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(mid_o + ((int64_t)b * num_q_heads + h) * num_splits * (kHeadDim + 1)), 0, 0x7FFFFFFF,
        0x00020000);
    // rows s0 .. s0 + 31 (rows past the last one, n_rows, re-read it: a cache hit)
    float l, v0[kMergeRows], v1[kMergeRows];
    auto load_chunk = [&](int s0, int n_rows) {
        l = lane < n_rows ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                           rows, (s0 + lane) * kRow + kHeadDim * 4, 0, 0))
                          : -INFINITY;
#pragma unroll
        for (int i = 0; i < kMergeRows; ++i) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(rows, (s0 + min(i, n_rows - 1)) * kRow + 8 * lane, 0, 0);
            // (elements copied out first: a bit cast applied to an element of the vector
            // in place reads element 0)
            const uint32_t x0 = v[0], x1 = v[1];
            v0[i] = __builtin_bit_cast(float, x0);
            v1[i] = __builtin_bit_cast(float, x1);
        }
    };
    load_chunk(0, min(kMergeRows, num_splits));
    const int seq_len = seq_lens[b];
    const int split_len = (seq_len + num_splits - 1) / num_splits;
    // splits [0, live) are the non-empty ones: split s is non-empty iff s * len < seq_len
    const int live = split_len > 0 ? min(num_splits, (seq_len + split_len - 1) / split_len) : 0;

    float mx = -INFINITY, a0 = 0.f, a1 = 0.f, wsum = 0.f;
    for (int s0 = 0; s0 < live; s0 += kMergeRows) {
        const int n = min(kMergeRows, live - s0);
        if (s0 > 0) {
            load_chunk(s0, n);
        } else {
            // the first chunk was loaded for all of its splits: drop the empty ones
            l = lane < n ? l : -INFINITY;
#pragma unroll
            for (int i = 0; i < kMergeRows; ++i) {
                v0[i] = i < n ? v0[i] : 0.f;
                v1[i] = i < n ? v1[i] : 0.f;
            }
        }
        const float m_new = fmaxf(mx, wave_max(l));
        const float scale = expf(mx - m_new);  // 0 for the first chunk (mx = -inf)
        const float w = expf(l - m_new);       // 0 on lanes past the chunk
        a0 *= scale;
        a1 *= scale;
        wsum = wsum * scale + wave_sum(w);
#pragma unroll
        for (int i = 0; i < kMergeRows; ++i) {
            const float wi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), i));
            a0 = fmaf(wi, v0[i], a0);
            a1 = fmaf(wi, v1[i], a1);
        }
        mx = m_new;
    }
    const float inv = 1.f / wsum;
    OutT *o = out + ((int64_t)b * num_q_heads + h) * kHeadDim;
    o[2 * lane] = from_float<OutT>(a0 * inv);
    o[2 * lane + 1] = from_float<OutT>(a1 * inv);
    if (lane == 0)
        lse[(int64_t)b * num_q_heads + h] = mx + logf(wsum);
}

// Rotation on the f16 matrix cores: q_rot = query @ rot_t with rot_t split into f16
// hi + lo parts (hi + lo = rot_t to ~2^-22), and for fp32 queries the query too
// (products hi*hi + hi*lo + lo*hi).  Each query row is first scaled by a power of two 2^e
// that puts its largest magnitude in [2^14, 2^15) -- inside the f16 range for any fp32 or
// bf16 row, and with the lo parts of the row's large elements out of f16 denormals -- and
// the result row is scaled back by 2^-e (both exact).  fp16 and bf16 rows are then exact in
// f16 (lo part 0) but for elements 2^29 times below the row's largest.  A workgroup of 4
// waves stages rot_t^T as f16 parts in LDS (2 x 32 KB) and each wave rotates 16 rows: lane
// (n, g) feeds A[row n][k 8g .. 8g+7] and B[k 8g .. 8g+7][col n] of
// v_mfma_f32_16x16x32_f16 and gets D[rows 4g .. 4g+3][col n].
constexpr int kRotWaves = 4;
constexpr int kRotMfmaRows = 16 * kRotWaves;  // rows per workgroup
constexpr int kRotPt = kHeadDim + 8;           // LDS row of rot_t^T (halves), 16-byte aligned
typedef _Float16 rot_half8 __attribute__((ext_vector_type(8)));

template <typename InT, typename V8>
__device__ __forceinline__ void rot_a_operands(const V8 &p, int e, rot_half8 &hi, rot_half8 &lo) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float x = __builtin_ldexpf(to_float<InT>(p[j]), e);
        hi[j] = (_Float16)x;
        lo[j] = sizeof(InT) == 4 ? (_Float16)(x - (float)hi[j]) : (_Float16)0.f;
    }
}

// Largest |x| of a query row over its four lanes n, n + 16, n + 32, n + 48.
// (The swap results are read by value before the bit cast: a bit cast of the returned
// vector's element lvalue reads its first element.)
__device__ __forceinline__ float rot_row_max(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    uint32_t a = r[0], b = r[1];
    x = fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
    const uint32_t v = __builtin_bit_cast(uint32_t, x);
    r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    a = r[0];
    b = r[1];
    return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}

template <typename InT>
__global__ __launch_bounds__(kWave *kRotWaves) void rotate_mfma_kernel(const InT *__restrict__ query,
                                                                        const float *__restrict__ rot_t,
                                                                        float *__restrict__ q_rot, int rows,
                                                                        const float *__restrict__ centroids,
                                                                        float *__restrict__ pair_lut) {
    __shared__ __align__(16) _Float16 pt_hi[kHeadDim * kRotPt];  // [col][k]
    __shared__ __align__(16) _Float16 pt_lo[kHeadDim * kRotPt];
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int n = lane & 15, g = lane >> 4;
    const int r0 = blockIdx.x * kRotMfmaRows + 16 * wave;
    // side task of the first workgroup: the pair LUT (row lo * 16 + hi = (c[lo], c[hi])),
    // loaded here and stored at the end, off the staging's critical path
    static_assert(kWave * kRotWaves == 256, "one thread per pair-LUT row");
    const bool lut_task = pair_lut && blockIdx.x == 0;
    float c_lo = 0.f, c_hi = 0.f;
    if (lut_task) {
        c_lo = centroids[threadIdx.x / 16];
        c_hi = centroids[threadIdx.x % 16];
    }
    // the query rows go out first (rows past the end repeat the last one, not stored)
    const int ra = min(r0 + n, rows - 1);
    // 8 consecutive elements per (kb, lane): 16-byte loads (the query is 16-byte aligned)
    typedef InT in8 __attribute__((ext_vector_type(8)));
    in8 qv[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
        qv[kb] = *reinterpret_cast<const in8 *>(query + (int64_t)ra * kHeadDim + 32 * kb + 8 * g);
    // thread (c, kg): rot_t[8kg .. 8kg+7][c] (coalesced over c) -> one 16-byte LDS write
    // into each part.  All 64 loads of a thread go out before the first conversion.
    constexpr int kIters = kHeadDim * (kHeadDim / 8) / (kWave * kRotWaves);
    float wv[kIters][8];
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
        const int i = threadIdx.x + it * kWave * kRotWaves;
        const int c = i % kHeadDim, kg = i / kHeadDim;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            wv[it][j] = rot_t[(8 * kg + j) * kHeadDim + c];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
        const int i = threadIdx.x + it * kWave * kRotWaves;
        const int c = i % kHeadDim, kg = i / kHeadDim;
        rot_half8 h, l;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            h[j] = (_Float16)wv[it][j];
            l[j] = (_Float16)(wv[it][j] - (float)h[j]);
        }
        *reinterpret_cast<rot_half8 *>(pt_hi + c * kRotPt + 8 * kg) = h;
        *reinterpret_cast<rot_half8 *>(pt_lo + c * kRotPt + 8 * kg) = l;
    }
    __syncthreads();
    if (lut_task) {
        pair_lut[2 * threadIdx.x] = c_lo;
        pair_lut[2 * threadIdx.x + 1] = c_hi;
    }
    if (r0 >= rows)
        return;
    // the row's scale 2^e: max |x| * 2^e in [2^14, 2^15) (e = 0 for a zero or non-finite max)
    float amax = 0.f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j)
            amax = fmaxf(amax, fabsf(to_float<InT>(qv[kb][j])));
    amax = rot_row_max(amax);
    const int e = (amax > 0.f && amax < __builtin_inff()) ? 15 - __builtin_amdgcn_frexp_expf(amax) : 0;
    // D row 4g + i is query row r0 + 4g + i, whose scale lane 4g + i (row n = 4g + i) holds
    int e_out[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        e_out[i] = __shfl(e, 4 * g + i, kWave);
    rot_half8 a_hi[4], a_lo[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
        rot_a_operands<InT>(qv[kb], e, a_hi[kb], a_lo[kb]);
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) {
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const int off = (16 * cb + n) * kRotPt + 32 * kb + 8 * g;
            const rot_half8 b_hi = *reinterpret_cast<const rot_half8 *>(pt_hi + off);
            const rot_half8 b_lo = *reinterpret_cast<const rot_half8 *>(pt_lo + off);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_hi[kb], b_hi, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_hi[kb], b_lo, acc, 0, 0, 0);
            if constexpr (sizeof(InT) == 4)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_lo[kb], b_hi, acc, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = r0 + 4 * g + i;
            if (r < rows)
                q_rot[(int64_t)r * kHeadDim + 16 * cb + n] = __builtin_ldexpf(acc[i], -e_out[i]);
        }
    }
}

__global__ void pair_lut_kernel(const float *__restrict__ cents, float *__restrict__ lut, int n) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t < n * n) {
        lut[2 * t] = cents[t / n];
        lut[2 * t + 1] = cents[t % n];
    }
}

}  // namespace tq4
