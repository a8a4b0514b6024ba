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
// 134-byte slot (t, h) = K bytes | fp16 norm | V bytes | fp16 scale | fp16 min, at byte
// t * slot_pos + h * slot_head of its block (position-major or head-major blocks; the
// reference's stride_cache_pos / stride_cache_head, reference/aos_store.py:375-377).
//
// A workgroup of 8 waves stages 16 * PiT^T in LDS as f16 hi + lo parts once, then its
// waves walk the rows 16 at a time (grid-stride); the first tile's K and V loads are issued
// right after the staging's own loads, each later tile's at the end of the previous one
// (fp32 V, 32 VGPRs, where it is used).  Lane (n, g) = (lane % 16, lane / 16) loads dims 32g .. 32g+31 of
// row n of K and V.  The rotation is the transposed product
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
//
// Bucketize: the workgroup builds a cell table over the midpoints' span (kCells cells of
// width w, about two spare cells each side, centred on y0 + kw with y0 = K w for an integer
// K).  Cell k's window is [y0 + (k - 1/2)w - w/64, y0 + (k + 1/2)w + w/64]; its entry holds
// the one midpoint inside the window (NaN if none), the number of midpoints below the
// window, and c^2 at those two indices.  The cell of y is round(y / w - K), read straight
// from the bits of fma(y, 1/w, 1.5 * 2^23 - K) (the bias leaves the rounded integer in the
// low mantissa bits) after a clamp to the table; a y whose computed cell is k lies inside
// window k (the computed coordinate is off by < 1e-3 cells for |y| <= 1; beyond the span the
// edge cells hold for every y), so count(midpoints <= y) = base + (y >= mid): one LDS read
// and one compare per element instead of 15.  When some window holds two midpoints (a
// codebook with a gap under ~w) the kernel counts all 15 instead.
//
// V codes: (v - min) * (1 / scale) is within 2^-18 of the fp32 quotient (v - min) / scale
// for quotients below 16, so the code (truncation of quotient + 0.5) is the same unless
// quotient + 0.5 lies within 2^-16 of an integer; such elements take the division (bf16
// inputs put ~0.2 % of quotients exactly on a half-integer: a per-element branch, since
// nearly every wave holds one).
#pragma once
#include "tq4_device.h"

namespace tq4 {
namespace store {

constexpr int kWaves = 8;           // waves per workgroup (launches of up to kSmallTiles tiles: 4)
constexpr int kSmallWaves = 4;
constexpr int kSmallTiles = 1024;   // 4-wave workgroups up to this many tiles: at most one per CU
constexpr int kRows = 16;           // rows per wave step
constexpr int kMaxGroups = 512;     // two resident workgroups per CU (LDS), 4 waves per SIMD
constexpr int kCells = 128;         // bucketize table cells
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

// 32 consecutive elements of one row as raw 16-byte words (16-byte aligned source).
template <class T> struct Chunk {
    uint4 u[2 * sizeof(T)];
};
template <class T> __device__ __forceinline__ void load_raw(Chunk<T> &c, const T *p, bool ok) {
    if (ok) {
#pragma unroll
        for (int i = 0; i < 2 * (int)sizeof(T); ++i)
            c.u[i] = reinterpret_cast<const uint4 *>(p)[i];
    } else {
#pragma unroll
        for (int i = 0; i < 2 * (int)sizeof(T); ++i)
            c.u[i] = uint4{0u, 0u, 0u, 0u};
    }
}
template <class T> __device__ __forceinline__ void to_floats(float (&x)[32], const Chunk<T> &c) {
#pragma unroll
    for (int i = 0; i < 2 * (int)sizeof(T); ++i) {
        const uint32_t w[4] = {c.u[i].x, c.u[i].y, c.u[i].z, c.u[i].w};
#pragma unroll
        for (int e = 0; e < 16 / (int)sizeof(T); ++e) {
            if constexpr (sizeof(T) == 4)
                x[4 * i + e] = __builtin_bit_cast(float, w[e]);
            else
                x[8 * i + e] = (float)__builtin_bit_cast(T, (uint16_t)(w[e / 2] >> (16 * (e % 2))));
        }
    }
}

__device__ __forceinline__ uint16_t half_bits(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
}

// Code j of a lane's 32 dims at B bits per code, least significant bit first (code j at
// bits [B*j, B*j + B) of the words w); j is a constant after unrolling.
template <int B, int N> __device__ __forceinline__ void put_code(uint32_t (&w)[N], int j, uint32_t c) {
    const int bit = B * j, wi = bit >> 5, sh = bit & 31;
    w[wi] |= c << sh;
    if (sh + B > 32)
        w[wi + 1] |= c >> (32 - sh);
}

// 2-byte stores of N words at a 2-byte aligned address.
template <int N> __device__ __forceinline__ void store_words_a2(uint8_t *p, const uint32_t (&w)[N]) {
    uint16_t *h = reinterpret_cast<uint16_t *>(p);
#pragma unroll
    for (int i = 0; i < N; ++i) {
        h[2 * i] = (uint16_t)(w[i] & 0xFFFFu);
        h[2 * i + 1] = (uint16_t)(w[i] >> 16);
    }
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

// V of one row chunk (the lane's 32 dims; the row's four lanes n + 16g reduce together) at
// VB bits: top = 2^VB - 1, scale = max((max - min) / top, 1e-8), code = clamp(int((v - min) /
// scale + 0.5), 0, top), packed at VB bits per code (4 bits: element j at bits 4(j % 8) of
// word j / 8).  The product with the reciprocal is within 2^-18 of the fp32 quotient for
// quotients below 16, so the code only differs when quotient + 0.5 lies within 2^-16 of an
// integer: those elements take the division.
//
// 4-bit codes take a shorter path.  q = v * rs + (-min * rs) in one fma differs from the real
// quotient R = (v - min) / scale by at most 15 * 2^-23 (rs, 1 ulp) + |min * rs| * 2^-24 (the
// rounded addend) + 2^-20 (the fma's rounding), and the fp32 quotient + 0.5 from R + 0.5 by
// at most 2^-19 + 2^-20: together under e = 2^-17 + |min * rs| * 2^-24.  Where q lies further
// than 2e from every half-integer, round-to-nearest(q) = trunc(R + 0.5) = the code, and
// v_cvt_pk_u8_f32 (round to nearest even, saturating to 0..255, NaN to 0) rounds q and packs
// it into a byte in one instruction; even and odd elements fill two words of bytes that one
// shift-or merges into nibbles.  The other elements take the division as above.
template <int VB = 4>
__device__ __forceinline__ void quantize_v(const float (&x)[32], uint32_t (&vw)[VB], float &scale, float &vmin) {
    constexpr int kTop = (1 << VB) - 1;
    float lo = x[0], hi = x[0];
#pragma unroll
    for (int i = 1; i < 32; ++i) {
        lo = fminf(lo, x[i]);
        hi = fmaxf(hi, x[i]);
    }
    vmin = row_min(lo);
    const float vmax = row_max(hi);
    scale = (vmax - vmin) / (float)kTop;
    scale = scale > 1e-8f ? scale : 1e-8f;
    const float rs = __builtin_amdgcn_rcpf(scale);  // 1 ulp: the 2^-18 bound above holds
    if constexpr (VB == 4) {
        const float nb = -vmin * rs;
        // |q - rint(q)| below lim: q is more than 2e from the half-integers (NaN: no branch,
        // code 0 as the division's path gives)
        const float lim = 0.5f - (0x1p-16f + fabsf(nb) * 0x1p-22f);
        uint32_t ev[4] = {0u, 0u, 0u, 0u}, od[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            float q = fmaf(x[j], rs, nb);
            if (fabsf(q - rintf(q)) >= lim) {  // near a code boundary: the division
                asm volatile("");
                q = fminf(floorf((x[j] - vmin) / scale + 0.5f), (float)kTop);
            }
            uint32_t &w = (j & 1) ? od[j / 8] : ev[j / 8];
            w = __builtin_amdgcn_cvt_pk_u8_f32(q, (j % 8) / 2, w);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            vw[i] = ev[i] | (od[i] << 4);
        return;
    }
#pragma unroll
    for (int q = 0; q < VB; ++q)
        vw[q] = 0u;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        float f = (x[j] - vmin) * rs + 0.5f;
        if (fabsf(f - rintf(f)) < 0x1p-16f) {  // near a code boundary: the division
            asm volatile("");                   // (keeps it behind the branch)
            f = (x[j] - vmin) / scale + 0.5f;
        }
        const int c = (int)f;
        put_code<VB>(vw, j, (uint32_t)(c < 0 ? 0 : (c > kTop ? kTop : c)));
    }
}

// KB / VB: bits per K index / V code -- 4 / 4 is the turboquant_4bit_nc layout above;
// 3 / 4 (turboquant_k3v4_nc) and 3 / 3 (turboquant_3bit_nc) pack 8 codes in 3 bytes
// (reference/soa_store.py:319-337, :47-83): SoA record 16 KB + 16 VB bytes, AoS slot
// K | norm | V | scale | zero padded to even, written with 2-byte stores.
// W: waves per workgroup.  8 for large launches (two workgroups per CU share the CU's LDS,
// 4 waves per SIMD); 4 for launches of at most kSmallTiles tiles (a decode step's few
// rows), so that the waves spread over twice the CUs at one wave per SIMD: a wave's tile
// arithmetic then has its SIMD to itself, at the price of staging twice the PiT share.
template <int LAYOUT, class T, int KB = 4, int VB = 4, int W = kWaves>
__global__ __launch_bounds__(kWave *W) __attribute__((amdgpu_waves_per_eu(W == kWaves ? 4 : 1))) void store_kernel(
    const T *__restrict__ key, const T *__restrict__ value, const int32_t *__restrict__ slot_mapping,
    const float *__restrict__ pit, const float *__restrict__ midpoints, const float *__restrict__ centroids,
    uint8_t *__restrict__ cache, int rows, int num_kv_heads, int block_size, int64_t block_stride,
    int slot_pos, int slot_head, int norm_correction) {
    __shared__ __align__(16) _Float16 pt_hi[kHeadDim * kHeadDim];
    __shared__ __align__(16) _Float16 pt_lo[kHeadDim * kHeadDim];
    constexpr int kMids = (1 << KB) - 1;  // Lloyd-Max midpoints
    __shared__ float c2tab[16];
    __shared__ __align__(16) float4 btab[kCells];
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int n = lane & 15, g = lane >> 4;
    const int tiles = (rows + kRows - 1) / kRows;
    const int stride = gridDim.x * W;
    int tile = blockIdx.x * W + wave;

    // Every workgroup reads PiT, the midpoints and the centroids (L2 hits after the first
    // workgroup): their loads go out ahead of the first tile's K and V.  Those reads, across
    // the grid, keep HBM busy for microseconds, and a staging load queued behind them would
    // hold the workgroup's staging, and with it every wave's first tile, until they drain.
    // (centroids may be null without norm correction: read only with it)
    constexpr int kCents = 1 << KB;
    float mid[kMids], cent[kCents];
#pragma unroll
    for (int i = 0; i < kMids; ++i)
        mid[i] = midpoints[i];
#pragma unroll
    for (int i = 0; i < kCents; ++i)
        cent[i] = 0.f;
    if (norm_correction) {
#pragma unroll
        for (int i = 0; i < kCents; ++i)
            cent[i] = centroids[i];
    }
    // thread (c, k8): 16 * PiT[8k8 .. 8k8+7][c] (coalesced over c) -> one 16-byte LDS write
    // into each part
    constexpr int kStage = kHeadDim * (kHeadDim / 8) / (kWave * W);
    float pw[kStage][8];
#pragma unroll
    for (int it = 0; it < kStage; ++it) {
        const int i = threadIdx.x + it * kWave * W;
        const int c = i % kHeadDim, k8 = i / kHeadDim;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            pw[it][j] = pit[(8 * k8 + j) * kHeadDim + c];
    }
    __builtin_amdgcn_sched_barrier(0);
    constexpr bool kEarlyV = sizeof(T) < 4;
    Chunk<T> kr, vr;
    {
        const int64_t row = (int64_t)tile * kRows + n;
        load_raw(kr, key + row * kHeadDim + 32 * g, row < rows);
        if constexpr (kEarlyV)
            load_raw(vr, value + row * kHeadDim + 32 * g, row < rows);
    }
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (int it = 0; it < kStage; ++it) {
        const int i = threadIdx.x + it * kWave * W;
        const int c = i % kHeadDim, k8 = i / kHeadDim;
        half8 h, l;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float w = 16.f * pw[it][j];
            h[j] = (_Float16)w;
            l[j] = (_Float16)(w - (float)h[j]);
        }
        *reinterpret_cast<half8 *>(pt_hi + pt_off(c, k8)) = h;
        *reinterpret_cast<half8 *>(pt_lo + pt_off(c, k8)) = l;
    }
    // c[idx]^2 (0 without norm correction) of a lane's index, selected from the registers
    auto c2_at = [&](int idx) {
        float r = 0.f;
#pragma unroll
        for (int i = 0; i < kCents; ++i)
            r = idx == i ? cent[i] * cent[i] : r;
        return norm_correction ? r : 0.f;
    };
    if (threadIdx.x <= kMids)
        c2tab[threadIdx.x] = c2_at(threadIdx.x);
    float mmin = mid[0], mmax = mid[0];
#pragma unroll
    for (int i = 1; i < kMids; ++i) {
        mmin = fminf(mmin, mid[i]);
        mmax = fmaxf(mmax, mid[i]);
    }
    const float w = (mmax - mmin) / (float)(kCells - 4);
    // cells centred on y0 + kw, y0 = K w with K an integer: the cell coordinate y / w - K
    // then needs no fractional offset, and the 1.5 * 2^23 bias rounds it in the same fma
    const float kcell = floorf((mmin - 2.f * w) / w);
    const float y0 = kcell * w;
    // the cell coordinate's rounding error grows like (|K| + 128) 2^-23 cells against the
    // w / 64 widening of the windows: midpoints far from zero relative to their span (|K| >=
    // 2^14; Lloyd-Max codebooks have |K| ~ 66) take the counting path
    int cell_ok = fabsf(kcell) < 0x1p14f;
    if (threadIdx.x < kCells) {
        const int k = threadIdx.x;
        const float lo = y0 + ((float)k - 0.5f) * w - w * (1.f / 64), hi = y0 + ((float)k + 0.5f) * w + w * (1.f / 64);
        int base = 0, inside = 0;
        float m_in = __builtin_nanf("");  // compares false with every y
#pragma unroll
        for (int i = 0; i < kMids; ++i) {
            base += mid[i] < lo ? 1 : 0;
            if (mid[i] >= lo && mid[i] <= hi) {
                ++inside;
                m_in = mid[i];
            }
        }
        cell_ok = cell_ok && inside <= 1 && w > 0.f && w < __builtin_inff();
        const int up = base < kMids ? base + 1 : kMids;
        // the midpoint is stored x 256, the scale of the rotation's results
        btab[k] = float4{256.f * m_in, __builtin_bit_cast(float, base), c2_at(base), c2_at(up)};
    }
    const bool use_cells = __syncthreads_and(cell_ok) != 0;
    // biased cell coordinate y / w - K + 1.5 * 2^23 of y = acc / 256
    constexpr float kBias = 12582912.f;  // 1.5 * 2^23: the sum's low mantissa bits hold the rounded value
    const float inv_w = (1.f / w) * (1.f / 256.f), c0 = kBias - kcell;

    for (; tile < tiles; tile += stride) {
        const int row = tile * kRows + n;
        const bool in_range = row < rows;
        const int tok = in_range ? row / num_kv_heads : 0;
        const int head = in_range ? row % num_kv_heads : 0;
        const int64_t nrow = (int64_t)(tile + stride) * kRows + n;  // next tile of this wave

        // K: norm and x_hat of the lane's 32 dims
        float x[32];
        to_floats(x, kr);
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i)
            ss = fmaf(x[i], x[i], ss);
        const float norm = sqrtf(row_sum(ss));
        // x_hat * 16 (16 is an exact power-of-two scale)
        const float rn = 16.f / (norm + 1e-8f);
        half8 b_hi[4], b_lo[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                // v as one fp32 register value: otherwise the compiler may fold the product
                // into one of the f16 casts (v_fma_mix, a single rounding) and not the other, and
                // where the two roundings differ (the fp32 product on an f16 tie) hi + lo is off
                // by an f16 ulp of x_hat * 16
                float v = x[8 * kb + j] * rn;
                asm("" : "+v"(v));
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
        // lane (n, g): acc[j / 4][j % 4] = 256 * y[row n][32g + j]
        // K indices at KB bits (4 bits: element j at bits 4(j % 8) of word j / 8)
        uint32_t kw[KB];
#pragma unroll
        for (int q = 0; q < KB; ++q)
            kw[q] = 0u;
        float csq = 0.f;
        if (use_cells) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
#pragma unroll
                for (int j = 8 * q; j < 8 * q + 8; ++j) {
                    const float a = acc[j / 4][j % 4];
                    const float t = fminf(fmaxf(fmaf(a, inv_w, c0), kBias), kBias + (float)(kCells - 1));
                    const float4 e = btab[__builtin_bit_cast(int, t) - __builtin_bit_cast(int, kBias)];
                    const bool ge = a >= e.x;
                    put_code<KB>(kw, j, (uint32_t)(__builtin_bit_cast(int, e.y) + (ge ? 1 : 0)));
                    csq += ge ? e.w : e.z;
                }
                // at most 8 table reads in flight (32 VGPRs)
                asm volatile("" ::: "memory");
            }
        } else {
#pragma unroll
            for (int j = 0; j < 32; ++j) {
                const float y = acc[j / 4][j % 4] * (1.f / 256.f);
                int c = 0;
#pragma unroll
                for (int i = 0; i < kMids; ++i)
                    c += y >= mid[i] ? 1 : 0;
                put_code<KB>(kw, j, (uint32_t)c);
                csq += c2tab[c];
            }
        }
        const float csum = row_sum(csq);
        const float kscalar = norm_correction ? norm * (1.0f / sqrtf(csum + 1e-16f)) : norm;

        // V: per-row min / max, uniform 4-bit codes
        if constexpr (!kEarlyV)
            load_raw(vr, value + (int64_t)row * kHeadDim + 32 * g, in_range);
        to_floats(x, vr);
        float scale, vmin;
        uint32_t vw[VB];
        quantize_v<VB>(x, vw, scale, vmin);
        const int slot = in_range ? slot_mapping[tok] : -1;
        if (KB != 4 || VB != 4) {
            if (slot >= 0) {
                const int64_t blk = slot / block_size, off = slot % block_size;
                uint8_t *base = cache + blk * block_stride;
                constexpr int kK = 16 * KB, kV = 16 * VB;
                if constexpr (LAYOUT == 0) {
                    uint8_t *rec = base + (off * num_kv_heads + head) * (kK + kV);
                    store_words_a2(rec + 4 * KB * g, kw);
                    store_words_a2(rec + kK + 4 * VB * g, vw);
                    if (g == 0) {
                        uint16_t *meta = reinterpret_cast<uint16_t *>(base + (int64_t)block_size * num_kv_heads * (kK + kV)) +
                                         (int64_t)head * 3 * block_size + off;
                        meta[0] = half_bits(kscalar);
                        meta[block_size] = half_bits(scale);
                        meta[2 * block_size] = half_bits(vmin);
                    }
                } else {
                    uint8_t *sl = base + off * slot_pos + (int64_t)head * slot_head;
                    store_words_a2(sl + 4 * KB * g, kw);
                    store_words_a2(sl + kK + 2 + 4 * VB * g, vw);
                    if (g == 0) {
                        reinterpret_cast<uint16_t *>(sl + kK)[0] = half_bits(kscalar);
                        reinterpret_cast<uint16_t *>(sl + kK + 2 + kV)[0] = half_bits(scale);
                        reinterpret_cast<uint16_t *>(sl + kK + 4 + kV)[0] = half_bits(vmin);
                    }
                }
            }
        } else if (slot >= 0) {
            const int64_t blk = slot / block_size, off = slot % block_size;
            uint8_t *base = cache + blk * block_stride;
            const uint4 kb = uint4{kw[0], kw[KB > 1 ? 1 : 0], kw[KB > 2 ? 2 : 0], kw[KB > 3 ? 3 : 0]},
                        vb = uint4{vw[0], vw[VB > 1 ? 1 : 0], vw[VB > 2 ? 2 : 0], vw[VB > 3 ? 3 : 0]};
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
                uint8_t *sl = base + off * slot_pos + (int64_t)head * slot_head;
                store16_a2(sl + 16 * g, kb);
                store16_a2(sl + kHalfD + 2 + 16 * g, vb);
                if (g == 0) {
                    reinterpret_cast<uint16_t *>(sl + kHalfD)[0] = half_bits(kscalar);
                    reinterpret_cast<uint16_t *>(sl + kHeadDim + 2)[0] = half_bits(scale);
                    reinterpret_cast<uint16_t *>(sl + kHeadDim + 4)[0] = half_bits(vmin);
                }
            }
        }
        // the next tile of this wave
        load_raw(kr, key + nrow * kHeadDim + 32 * g, nrow < rows);
        if constexpr (kEarlyV)
            load_raw(vr, value + nrow * kHeadDim + 32 * g, nrow < rows);
    }
}

// FP8-key preset writer (reference/soa_store.py:125-212): K cast to E4M3 bytes (round to
// nearest even, saturating at +-448 as the reference's satfinite cast; NaN stays NaN), V as
// above.  SoA record (t, h) = 128 K bytes | 64 V bytes, metadata [h][field][t] with two
// fields (V scale, V zero); AoS slot = 128 K | 64 V | scale | zero (196 bytes, 4-byte
// aligned: dword stores).  A wave takes 16 rows; lane (n, g) = row n, dims 32g .. 32g+31.
constexpr int kFp8Waves = 4;
constexpr int kFp8Record = kHeadDim + kHalfD;
__device__ __forceinline__ float sat_e4m3(float x) {
    return x > 448.f ? 448.f : (x < -448.f ? -448.f : x);  // comparisons keep NaN
}
template <int LAYOUT, class T>
__global__ __launch_bounds__(kWave *kFp8Waves) void store_fp8_kernel(const T *__restrict__ key,
                                                                     const T *__restrict__ value,
                                                                     const int32_t *__restrict__ slot_mapping,
                                                                     uint8_t *__restrict__ cache, int rows,
                                                                     int num_kv_heads, int block_size,
                                                                     int64_t block_stride, int slot_pos,
                                                                     int slot_head) {
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int n = lane & 15, g = lane >> 4;
    const int tiles = (rows + kRows - 1) / kRows;
    for (int tile = blockIdx.x * kFp8Waves + wave; tile < tiles; tile += gridDim.x * kFp8Waves) {
        const int row = tile * kRows + n;
        const bool in_range = row < rows;
        Chunk<T> kr, vr;
        load_raw(kr, key + (int64_t)row * kHeadDim + 32 * g, in_range);
        load_raw(vr, value + (int64_t)row * kHeadDim + 32 * g, in_range);
        float x[32];
        to_floats(x, kr);
        uint32_t kw[8];  // dims 32g + 4i .. 32g + 4i + 3, low byte first
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            int p = __builtin_amdgcn_cvt_pk_fp8_f32(sat_e4m3(x[4 * i]), sat_e4m3(x[4 * i + 1]), 0, false);
            p = __builtin_amdgcn_cvt_pk_fp8_f32(sat_e4m3(x[4 * i + 2]), sat_e4m3(x[4 * i + 3]), p, true);
            kw[i] = (uint32_t)p;
        }
        to_floats(x, vr);
        float scale, vmin;
        uint32_t vw[4];
        quantize_v<4>(x, vw, scale, vmin);
        const int tok = in_range ? row / num_kv_heads : 0;
        const int head = in_range ? row % num_kv_heads : 0;
        const int slot = in_range ? slot_mapping[tok] : -1;
        if (slot < 0)
            continue;
        const int64_t blk = slot / block_size, off = slot % block_size;
        uint8_t *base = cache + blk * block_stride;
        uint32_t *r = reinterpret_cast<uint32_t *>(
            base + (LAYOUT == 0 ? (off * num_kv_heads + head) * kFp8Record : off * slot_pos + (int64_t)head * slot_head));
#pragma unroll
        for (int i = 0; i < 8; ++i)
            r[8 * g + i] = kw[i];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            r[kHeadDim / 4 + 4 * g + i] = vw[i];
        if (g == 0) {
            uint16_t *f;
            int fstride;
            if constexpr (LAYOUT == 0) {
                f = reinterpret_cast<uint16_t *>(base + (int64_t)block_size * num_kv_heads * kFp8Record) +
                    (int64_t)head * 2 * block_size + off;
                fstride = block_size;
            } else {
                f = reinterpret_cast<uint16_t *>(reinterpret_cast<uint8_t *>(r) + kFp8Record);
                fstride = 1;
            }
            f[0] = half_bits(scale);
            f[fstride] = half_bits(vmin);
        }
    }
}

}  // namespace store
}  // namespace tq4
