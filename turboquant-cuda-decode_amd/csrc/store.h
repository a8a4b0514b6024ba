// Cache writer for the TurboQuant 4-bit cache (the write side of the decode path's data
// format), gfx950.
//
// Per (token, kv-head) row, as reference/soa_store.py:381-524 (launcher: norm, x_hat and
// the rotation GEMM) and :223-380 (bucketize, pack, norm, value quantization) do in two
// steps, here fused in one kernel:
//   K: norm = ||k||, x_hat = k / (norm + 1e-8), y = x_hat @ PiT, idx_d = number of
//      Lloyd-Max midpoints <= y_d, two 4-bit indices per byte (low nibble = even dim);
//      stored scalar fp16(norm / sqrt(sum c[idx]^2 + 1e-16)) (norm correction) or
//      fp16(norm);
//   V: scale = max((max - min) / 15, 1e-8), code = clamp(int((v - min) / scale + 0.5),
//      0, 15), fp16 scale and fp16 min.
// SoA: codes in the block's data region (record (t, h) = 64 K bytes then 64 V bytes),
// the three fp16 scalars in its metadata region [h][field][t].  AoS (reference/aos_store.py):
// 134-byte slot (t, h) = K bytes | fp16 norm | V bytes | fp16 scale | fp16 min.
//
// A workgroup of 8 waves stages 16 * PiT^T in LDS as f16 hi + lo parts once, then its
// waves walk the rows 16 at a time (grid-stride).  Lane (n, g) = (lane % 16, lane / 16)
// loads dims 32g .. 32g+31 of row n of K and V.  The rotation is the transposed product
// y^T = PiT^T x_hat^T on v_mfma_f32_16x16x32_f16, with operands and x_hat (scaled by 16,
// keeping the lo parts out of f16 denormals) split into f16 hi + lo (products hi*hi +
// hi*lo + lo*hi, ~fp32 accurate).  Two index maps make every operand and result
// lane-local:
//   contraction: step kb, MFMA k-index 8g + j  <->  dim 32g + 8kb + j, so lane (n, g)'s
//                B operand is 8 of its own loaded x_hat values;
//   output:      MFMA row r of column block cb <-> dim 32(r/4) + 4cb + r%4, so the D
//                registers of lane (n, g) are y[row n][32g + 4cb + i] -- its own 32 dims
//                in order, ready for bucketize and packing.
// Reductions over a row's four lanes (n + 16g) use permlane swaps.
#pragma once
#include "tq4_device.h"

namespace tq4 {
namespace store {

constexpr int kWaves = 8;           // waves per workgroup
constexpr int kRows = 16;           // rows per wave step
constexpr int kMaxGroups = 512;     // 2 resident workgroups per CU (64 KB LDS each)
typedef _Float16 half8 __attribute__((ext_vector_type(8)));

// LDS image of PiT^T: row c (an output dim) holds PiT[0 .. 127][c] as 16 chunks of 8
// halves, chunk k8 at position k8 ^ swz(c).  The 16 rows one 16-lane group reads at a time
// (c = 32m + 4cb + i, m, i = 0..3) then hit 16 different chunk positions: all 64 banks.
__device__ __forceinline__ int swz(int c) { return (c & 3) | ((c >> 3) & 12); }
__device__ __forceinline__ int pt_off(int c, int k8) { return c * kHeadDim + 8 * (k8 ^ swz(c)); }

__device__ __forceinline__ uint32_t fbits(float x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ float bitsf(uint32_t x) { return __builtin_bit_cast(float, x); }
// Sum / min / max over the four lanes n, n+16, n+32, n+48.
__device__ __forceinline__ float row_sum(float x) {
    auto r = __builtin_amdgcn_permlane16_swap(fbits(x), fbits(x), false, false);
    x = bitsf(r[0]) + bitsf(r[1]);
    r = __builtin_amdgcn_permlane32_swap(fbits(x), fbits(x), false, false);
    return bitsf(r[0]) + bitsf(r[1]);
}
__device__ __forceinline__ float row_min(float x) {
    auto r = __builtin_amdgcn_permlane16_swap(fbits(x), fbits(x), false, false);
    x = fminf(bitsf(r[0]), bitsf(r[1]));
    r = __builtin_amdgcn_permlane32_swap(fbits(x), fbits(x), false, false);
    return fminf(bitsf(r[0]), bitsf(r[1]));
}
__device__ __forceinline__ float row_max(float x) {
    auto r = __builtin_amdgcn_permlane16_swap(fbits(x), fbits(x), false, false);
    x = fmaxf(bitsf(r[0]), bitsf(r[1]));
    r = __builtin_amdgcn_permlane32_swap(fbits(x), fbits(x), false, false);
    return fmaxf(bitsf(r[0]), bitsf(r[1]));
}

// 32 consecutive elements as fp32 (16-byte aligned source).
template <class T> __device__ __forceinline__ void load_chunk(float (&x)[32], const T *p) {
    if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 v = reinterpret_cast<const float4 *>(p)[i];
            x[4 * i] = v.x;
            x[4 * i + 1] = v.y;
            x[4 * i + 2] = v.z;
            x[4 * i + 3] = v.w;
        }
    } else {
        typedef T t8 __attribute__((ext_vector_type(8)));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const t8 v = reinterpret_cast<const t8 *>(p)[i];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                x[8 * i + j] = (float)v[j];
        }
    }
}

__device__ __forceinline__ uint16_t half_bits(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
}

// Two 4-bit codes per byte, low nibble = even element: 32 codes -> 16 bytes.
__device__ __forceinline__ uint4 pack32(const int (&c)[32]) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t v = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            v |= (uint32_t)((c[8 * i + 2 * j] & 15) | ((c[8 * i + 2 * j + 1] & 15) << 4)) << (8 * j);
        w[i] = v;
    }
    return uint4{w[0], w[1], w[2], w[3]};
}

// 2-byte stores of 16 bytes at a 2-byte aligned address (AoS slots).
__device__ __forceinline__ void store16_a2(uint8_t *p, uint4 v) {
    uint16_t *h = reinterpret_cast<uint16_t *>(p);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h[2 * i] = (uint16_t)(w[i] & 0xFFFFu);
        h[2 * i + 1] = (uint16_t)(w[i] >> 16);
    }
}

template <int LAYOUT, class T>
__global__ __launch_bounds__(kWave *kWaves) void store_kernel(const T *__restrict__ key, const T *__restrict__ value,
                                                      const int32_t *__restrict__ slot_mapping,
                                                      const float *__restrict__ pit,
                                                      const float *__restrict__ midpoints,
                                                      const float *__restrict__ centroids,
                                                      uint8_t *__restrict__ cache, int rows, int num_kv_heads,
                                                      int block_size, int64_t block_stride,
                                                      int norm_correction) {
    __shared__ __align__(16) _Float16 pt_hi[kHeadDim * kHeadDim];
    __shared__ __align__(16) _Float16 pt_lo[kHeadDim * kHeadDim];
    __shared__ float c2tab[16];
    // thread (c, k8): 16 * PiT[8k8 .. 8k8+7][c] (coalesced over c) -> one 16-byte LDS write
    // into each part
#pragma unroll
    for (int it = 0; it < kHeadDim * (kHeadDim / 8) / (kWave * kWaves); ++it) {
        const int i = threadIdx.x + it * kWave * kWaves;
        const int c = i % kHeadDim, k8 = i / kHeadDim;
        half8 h, l;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float w = 16.f * pit[(8 * k8 + j) * kHeadDim + c];
            h[j] = (_Float16)w;
            l[j] = (_Float16)(w - (float)h[j]);
        }
        *reinterpret_cast<half8 *>(pt_hi + pt_off(c, k8)) = h;
        *reinterpret_cast<half8 *>(pt_lo + pt_off(c, k8)) = l;
    }
    if (threadIdx.x < 16)
        c2tab[threadIdx.x] = norm_correction ? centroids[threadIdx.x] * centroids[threadIdx.x] : 0.f;
    __syncthreads();
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int n = lane & 15, g = lane >> 4;

    float mid[15];
#pragma unroll
    for (int i = 0; i < 15; ++i)
        mid[i] = midpoints[i];

    const int tiles = (rows + kRows - 1) / kRows;
    for (int tile = blockIdx.x * kWaves + wave; tile < tiles; tile += gridDim.x * kWaves) {
        const int row = tile * kRows + n;
        const bool in_range = row < rows;
        const int tok = in_range ? row / num_kv_heads : 0;
        const int head = in_range ? row % num_kv_heads : 0;

        // K: norm and x_hat of the lane's 32 dims
        float x[32];
        if (in_range) {
            load_chunk(x, key + (int64_t)row * kHeadDim + 32 * g);
        } else {
#pragma unroll
            for (int i = 0; i < 32; ++i)
                x[i] = 0.f;
        }
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i)
            ss = fmaf(x[i], x[i], ss);
        const float norm = sqrtf(row_sum(ss));
        // x_hat * 16 (the division as written, then an exact power-of-two scale)
        half8 b_hi[4], b_lo[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float v = 16.f * (x[8 * kb + j] / (norm + 1e-8f));
                b_hi[kb][j] = (_Float16)v;
                b_lo[kb][j] = (_Float16)(v - (float)b_hi[kb][j]);
            }
        // column block cb: MFMA row r <-> dim 32(r/4) + 4cb + r%4 (lane (n, g) feeds row n).
        // The operand reads are the same for every tile; an opaque base keeps them in the loop
        // (hoisted, they would hold 256 VGPRs).
        int ldsb = 0;
        asm volatile("" : "+v"(ldsb));
        floatx4 acc[8];
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) {
            acc[cb] = floatx4{0.f, 0.f, 0.f, 0.f};
            const int c = 32 * (n >> 2) + 4 * cb + (n & 3);
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                const int off = ldsb + pt_off(c, 4 * g + kb);
                const half8 a_hi = *reinterpret_cast<const half8 *>(pt_hi + off);
                const half8 a_lo = *reinterpret_cast<const half8 *>(pt_lo + off);
                acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_hi, b_hi[kb], acc[cb], 0, 0, 0);
                acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_lo, b_hi[kb], acc[cb], 0, 0, 0);
                acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_hi, b_lo[kb], acc[cb], 0, 0, 0);
            }
        }
        // lane (n, g): acc[cb][i] = 256 * y[row n][32g + 4cb + i]
        float y[32];
#pragma unroll
        for (int cb = 0; cb < 8; ++cb)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                y[4 * cb + i] = acc[cb][i] * (1.f / 256.f);
        int kidx[32];
        float csq = 0.f;
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            int c = 0;
#pragma unroll
            for (int i = 0; i < 15; ++i)
                c += y[j] >= mid[i] ? 1 : 0;
            kidx[j] = c;
            csq += c2tab[c];
        }
        const float csum = row_sum(csq);
        const float kscalar = norm_correction ? norm * (1.0f / sqrtf(csum + 1e-16f)) : norm;

        // V: per-row min / max, uniform 4-bit codes
        if (in_range) {
            load_chunk(x, value + (int64_t)row * kHeadDim + 32 * g);
        } else {
#pragma unroll
            for (int i = 0; i < 32; ++i)
                x[i] = 0.f;
        }
        float lo = x[0], hi = x[0];
#pragma unroll
        for (int i = 1; i < 32; ++i) {
            lo = fminf(lo, x[i]);
            hi = fmaxf(hi, x[i]);
        }
        const float vmin = row_min(lo), vmax = row_max(hi);
        float scale = (vmax - vmin) / 15.0f;
        scale = scale > 1e-8f ? scale : 1e-8f;
        int vcode[32];
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const int c = (int)((x[j] - vmin) / scale + 0.5f);
            vcode[j] = c < 0 ? 0 : (c > 15 ? 15 : c);
        }

        const int slot = in_range ? slot_mapping[tok] : -1;
        if (slot < 0)
            continue;
        const int64_t blk = slot / block_size, off = slot % block_size;
        uint8_t *base = cache + blk * block_stride;
        const uint4 kb = pack32(kidx), vb = pack32(vcode);
        if constexpr (LAYOUT == 0) {
            uint8_t *rec = base + (off * num_kv_heads + head) * kSoaRecord;
            *reinterpret_cast<uint4 *>(rec + 16 * g) = kb;
            *reinterpret_cast<uint4 *>(rec + kHalfD + 16 * g) = vb;
            if (g == 0) {
                uint16_t *meta = reinterpret_cast<uint16_t *>(base + (int64_t)block_size * num_kv_heads * kSoaRecord) +
                                 (int64_t)head * 3 * block_size + off;
                meta[0] = half_bits(kscalar);
                meta[block_size] = half_bits(scale);
                meta[2 * block_size] = half_bits(vmin);
            }
        } else {
            uint8_t *sl = base + (off * num_kv_heads + head) * kAosSlot;
            store16_a2(sl + 16 * g, kb);
            store16_a2(sl + kHalfD + 2 + 16 * g, vb);
            if (g == 0) {
                reinterpret_cast<uint16_t *>(sl + kHalfD)[0] = half_bits(kscalar);
                reinterpret_cast<uint16_t *>(sl + kHeadDim + 2)[0] = half_bits(scale);
                reinterpret_cast<uint16_t *>(sl + kHeadDim + 4)[0] = half_bits(vmin);
            }
        }
    }
}

}  // namespace store
}  // namespace tq4
