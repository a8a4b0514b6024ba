// Device-side helpers shared by the gfx950 decode kernels: cache addressing,
// fp16 metadata reads, wave64 reductions.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tq4 {

constexpr int kHeadDim = 128;               // D: the kernels are specialised for D = 128
constexpr int kHalfD = kHeadDim / 2;        // packed bytes of one 4-bit vector
constexpr int kSoaRecord = kHeadDim;        // SoA data record: K codes | V codes
constexpr int kAosSlot = kHeadDim + 6;      // AoS slot: K | norm | V | scale | zero
constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
// Output element types of the fused epilogue (the ABI's TQ4_F32 / TQ4_BF16 / TQ4_F16).
constexpr int kOutF32 = 0, kOutBf16 = 1, kOutF16 = 2;
constexpr float kLn2 = 0.6931471805599453f;

typedef float floatx4 __attribute__((ext_vector_type(4)));

// Split partition: L = ceil(len / S), split s covers [s*L, min(s*L + L, len)).
struct SplitRange {
    int start, end;
};
__device__ __forceinline__ SplitRange split_range(int seq_len, int num_splits, int sid) {
    const int len = (seq_len + num_splits - 1) / num_splits;
    const int s0 = len * sid;
    return {s0, min(s0 + len, seq_len)};
}

__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(bits16 & 0xFFFFu));
}

__device__ __forceinline__ float load_half(const uint8_t *p) {
    return half_bits_to_float(*reinterpret_cast<const unsigned short *>(p));
}

// 32-bit little-endian read at a 2-byte aligned address (AoS slots are 2-byte aligned).
__device__ __forceinline__ uint32_t load_u32_a2(const uint8_t *p) {
    const unsigned short *h = reinterpret_cast<const unsigned short *>(p);
    return (uint32_t)h[0] | ((uint32_t)h[1] << 16);
}

template <typename T> __device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1)
        v += __shfl_xor(v, m, kWave);
    return v;
}

template <typename T> __device__ __forceinline__ T wave_max(T v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1)
        v = fmaxf(v, __shfl_xor(v, m, kWave));
    return v;
}

// Byte address of the SoA data record of (block, token-in-block, kv-head).
__device__ __forceinline__ const uint8_t *soa_record(const uint8_t *cache, int64_t block,
                                                     int64_t stride, int off, int num_kv_heads,
                                                     int kvh) {
    return cache + block * stride + ((int64_t)off * num_kv_heads + kvh) * kSoaRecord;
}

// Byte address of fp16 metadata field f of (block, token-in-block, kv-head).
__device__ __forceinline__ const uint8_t *soa_meta(const uint8_t *cache, int64_t block,
                                                   int64_t stride, int off, int num_kv_heads,
                                                   int kvh, int block_size, int field) {
    return cache + block * stride + (int64_t)block_size * num_kv_heads * kSoaRecord +
           (((int64_t)kvh * 3 + field) * block_size + off) * 2;
}


}  // namespace tq4
