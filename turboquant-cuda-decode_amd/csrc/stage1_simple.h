// Stage1, plain-VALU kernel: one wave64 per (split, kv-head, sequence).
//
// Score phase: lane = token (64 tokens per tile).  Each lane decodes its token's
// 128 K codes through the 16-entry centroid table in LDS and accumulates the G
// head dots against q (LDS broadcast reads).  Online softmax in the exp2 domain
// with wave-wide max / sum per tile.
// Value phase: lane = dims (2*lane, 2*lane+1).  The tile's V code records are
// staged in LDS; acc[h][d] += (p_t * scale_t) * code_td, and sum_t p_t * zero_t is
// kept apart and added once at the end (v = code * scale + zero, and code * scale
// is exact in fp32).
//
// Covers any GQA group G <= 16 and any block size; it is the general fallback of
// the MFMA kernel and its cross-check on the GPU.  AoS slot (t, h) of a block starts at
// t * slot_pos + h * slot_head (position-major or head-major blocks); SoA ignores both.
#pragma once
#include "tq4_device.h"

namespace tq4 {

// Code d of a row packed at B bits per code, least significant bit first (code d at bits
// [B*d, B*d + B) of the byte string, read as little-endian words w); d is a constant after
// unrolling, so the word index and shifts are too.
template <int B> __device__ __forceinline__ uint32_t code_at(const uint32_t *w, int d) {
    const int bit = B * d, wi = bit >> 5, sh = bit & 31;
    uint32_t v = w[wi] >> sh;
    if (sh + B > 32)
        v |= w[wi + 1] << (32 - sh);
    return v & ((1u << B) - 1u);
}

// N little-endian words at p: 16-byte loads when p is 16-byte aligned (SoA records with a
// 16-byte block stride), else 2-byte loads (AoS slots are only 2-byte aligned).
template <int N> __device__ __forceinline__ void load_words(uint32_t (&w)[N], const uint8_t *p, bool a16) {
    static_assert(N % 4 == 0, "whole 16-byte chunks");
    if (a16) {
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {
            const uint4 v = reinterpret_cast<const uint4 *>(p)[i];
            w[4 * i] = v.x;
            w[4 * i + 1] = v.y;
            w[4 * i + 2] = v.z;
            w[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i)
            w[i] = load_u32_a2(p + 4 * i);
    }
}

// KF8: the FP8-key preset -- K is one E4M3 byte per dim (no codebook, no norm, the query
// is not rotated); record D + D/2 bytes (SoA; two metadata fields: V scale, V zero) or a
// D + D/2 + 4 byte slot (AoS: V scale and zero after the V codes).
// KB > 0: the KB-bit key / VB-bit value presets (turboquant_k3v4_nc, turboquant_3bit_nc,
// and 4/4), reference/config.py:20-40, with the codes packed at KB (VB) bits per dim
// (reference/soa_decode_v1.py:122-132, :271-284): record 16 KB + 16 VB bytes (SoA; three
// metadata fields: K norm, V scale, V zero) or a slot K | norm | V | scale | zero padded to
// even (AoS); the pair_lut argument then holds the 2^KB centroids themselves.
template <int LAYOUT, int G, bool KF8 = false, int KB = 0, int VB = 4>
__global__ __launch_bounds__(kWave) void stage1_simple_kernel(
    const float *__restrict__ q_rot, const uint8_t *__restrict__ cache,
    const int32_t *__restrict__ block_table, const int32_t *__restrict__ seq_lens,
    const float *__restrict__ pair_lut, float *__restrict__ mid_o, const float *__restrict__ sinks,
    int num_q_heads, int num_kv_heads, int block_size, int max_blocks, int64_t block_stride,
    int slot_pos, int slot_head, int num_splits, float score_scale_log2) {
    const int sid = blockIdx.x;
    const int kvh = blockIdx.y;
    const int b = blockIdx.z;
    const int lane = threadIdx.x;
    const SplitRange r = split_range(seq_lens[b], num_splits, sid);
    if (r.start >= r.end)
        return;

    __shared__ float lut[16];
    __shared__ float qs[G][kHeadDim];
    __shared__ float pw[G][kWave];
    __shared__ uint32_t vstage[kWave][kHalfD / 4 + 1];  // +1 word: bank spread

    if constexpr (KB > 0) {
        if (lane < (1 << KB))
            lut[lane] = pair_lut[lane];
    } else if (!KF8 && lane < 16) {
        lut[lane] = pair_lut[2 * (lane * 16)];  // row (lane, 0) = (c[lane], c[0])
    }
    for (int i = lane; i < G * kHeadDim; i += kWave) {
        const int h = i / kHeadDim, d = i % kHeadDim;
        qs[h][d] = q_rot[((int64_t)b * num_q_heads + kvh * G + h) * kHeadDim + d];
    }
    __syncthreads();

    float m[G], l[G], zl[G], acc[G][2];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        // split 0 with sinks starts from the head's sink logit: max = sink, sum = 1
        const bool sink = sinks && sid == 0;
        m[h] = sink ? sinks[(int64_t)kvh * G + h] * kLog2e : -INFINITY;
        l[h] = sink ? 1.f : 0.f;
        zl[h] = 0.f;
        acc[h][0] = acc[h][1] = 0.f;
    }
    const int32_t *bt = block_table + (int64_t)b * max_blocks;
    // SoA record sizes (128, 192, 112, 96 bytes) are multiples of 16 and the cache is 16-byte
    // aligned, so with a 16-byte block stride every record starts 16-byte aligned
    const bool a16 = LAYOUT == 0 && (block_stride & 15) == 0;

    for (int t0 = r.start; t0 < r.end; t0 += kWave) {
        const int t = t0 + lane;
        const bool valid = t < r.end;
        const int tc = valid ? t : r.end - 1;
        const int64_t blk = bt[tc / block_size];
        const int off = tc % block_size;
        const uint8_t *kp, *vp;
        float norm, vscale, vzero;
        constexpr int kKBytes = 16 * (KB > 0 ? KB : 4), kVBytes = 16 * VB;
        if constexpr (KB > 0) {
            if (LAYOUT == 0) {
                constexpr int rec = kKBytes + kVBytes;
                kp = cache + blk * block_stride + ((int64_t)off * num_kv_heads + kvh) * rec;
                vp = kp + kKBytes;
                const uint8_t *meta = cache + blk * block_stride + (int64_t)block_size * num_kv_heads * rec +
                                      ((int64_t)kvh * 3 * block_size + off) * 2;
                norm = load_half(meta);
                vscale = load_half(meta + 2 * block_size);
                vzero = load_half(meta + 4 * block_size);
            } else {
                kp = cache + blk * block_stride + (int64_t)off * slot_pos + (int64_t)kvh * slot_head;
                norm = load_half(kp + kKBytes);
                vp = kp + kKBytes + 2;
                vscale = load_half(vp + kVBytes);
                vzero = load_half(vp + kVBytes + 2);
            }
        } else if constexpr (KF8) {
            constexpr int rec = kHeadDim + kHalfD;
            if (LAYOUT == 0) {
                kp = cache + blk * block_stride + ((int64_t)off * num_kv_heads + kvh) * rec;
                const uint8_t *meta = cache + blk * block_stride + (int64_t)block_size * num_kv_heads * rec +
                                      ((int64_t)kvh * 2 * block_size + off) * 2;
                vscale = load_half(meta);
                vzero = load_half(meta + 2 * block_size);
            } else {
                kp = cache + blk * block_stride + (int64_t)off * slot_pos + (int64_t)kvh * slot_head;
                vscale = load_half(kp + rec);
                vzero = load_half(kp + rec + 2);
            }
            vp = kp + kHeadDim;
            norm = 1.f;
        } else if (LAYOUT == 0) {
            kp = soa_record(cache, blk, block_stride, off, num_kv_heads, kvh);
            vp = kp + kHalfD;
            norm = load_half(soa_meta(cache, blk, block_stride, off, num_kv_heads, kvh, block_size, 0));
            vscale = load_half(soa_meta(cache, blk, block_stride, off, num_kv_heads, kvh, block_size, 1));
            vzero = load_half(soa_meta(cache, blk, block_stride, off, num_kv_heads, kvh, block_size, 2));
        } else {
            kp = cache + blk * block_stride + (int64_t)off * slot_pos + (int64_t)kvh * slot_head;
            vp = kp + kHalfD + 2;
            norm = load_half(kp + kHalfD);
            vscale = load_half(kp + kHeadDim + 2);
            vzero = load_half(kp + kHeadDim + 4);
        }

        float s[G];
#pragma unroll
        for (int h = 0; h < G; ++h)
            s[h] = 0.f;
        float csq = 0.f;
        if constexpr (KB > 0) {
            uint32_t kw[4 * KB], vw[4 * VB];
            load_words(kw, kp, a16);
            load_words(vw, vp, a16);
#pragma unroll
            for (int d = 0; d < kHeadDim; ++d) {
                const float c = lut[code_at<KB>(kw, d)];
                if (LAYOUT == 1)
                    csq += c * c;
#pragma unroll
                for (int h = 0; h < G; ++h)
                    s[h] += qs[h][d] * c;
            }
#pragma unroll
            for (int w = 0; w < 4 * VB; ++w)
                vstage[lane][w] = vw[w];
        } else if constexpr (KF8) {
            uint32_t kw[kHeadDim / 4], vw[kHalfD / 4];
            load_words(kw, kp, a16);
            load_words(vw, vp, a16);
#pragma unroll
            for (int w = 0; w < kHeadDim / 4; ++w) {
                const uint32_t word = kw[w];
                const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)word, false);
                const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)word, true);
                const float k4[4] = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
                for (int n = 0; n < 4; ++n)
#pragma unroll
                    for (int h = 0; h < G; ++h)
                        s[h] += qs[h][4 * w + n] * k4[n];
            }
#pragma unroll
            for (int w = 0; w < kHalfD / 4; ++w)
                vstage[lane][w] = vw[w];
        } else {
            uint32_t kw[kHalfD / 4], vw[kHalfD / 4];
            load_words(kw, kp, a16);
            load_words(vw, vp, a16);
#pragma unroll
            for (int w = 0; w < kHalfD / 4; ++w) {
                const uint32_t word = kw[w];
#pragma unroll
                for (int n = 0; n < 8; ++n) {
                    const float c = lut[(word >> (4 * n)) & 15u];
                    if (LAYOUT == 1)
                        csq += c * c;
#pragma unroll
                    for (int h = 0; h < G; ++h)
                        s[h] += qs[h][8 * w + n] * c;
                }
                vstage[lane][w] = vw[w];
            }
        }
        float kscale = norm;
        if (!KF8 && LAYOUT == 1)
            kscale = norm * (1.0f / sqrtf(csq + 1e-16f));

#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float s2 = valid ? s[h] * kscale * score_scale_log2 : -INFINITY;
            const float mnew = fmaxf(m[h], wave_max(s2));  // finite: the tile has a valid token
            const float alpha = exp2f(m[h] - mnew);
            const float p = valid ? exp2f(s2 - mnew) : 0.f;
            l[h] = l[h] * alpha + wave_sum(p);
            zl[h] = zl[h] * alpha + (valid ? p * vzero : 0.f);
            acc[h][0] *= alpha;
            acc[h][1] *= alpha;
            m[h] = mnew;
            pw[h][lane] = valid ? p * vscale : 0.f;
        }
        __syncthreads();
        const int ntok = min(kWave, r.end - t0);
        for (int j = 0; j < ntok; ++j) {
            float c0, c1;
            if constexpr (VB == 4) {
                const uint32_t word = vstage[j][lane >> 2];
                const uint32_t byte = (word >> (8 * (lane & 3))) & 0xFFu;
                c0 = (float)(byte & 15u);
                c1 = (float)(byte >> 4);
            } else {
                // dims 2 lane, 2 lane + 1 at bits 2 VB lane .. 2 VB lane + 2 VB - 1 of the
                // record (a word pair; the second word may be the row's pad word, masked off)
                const int bit = 2 * VB * lane, wi = bit >> 5;
                const uint64_t win = (uint64_t)vstage[j][wi] | ((uint64_t)vstage[j][wi + 1] << 32);
                const uint32_t pair = (uint32_t)(win >> (bit & 31));
                c0 = (float)(pair & ((1u << VB) - 1u));
                c1 = (float)((pair >> VB) & ((1u << VB) - 1u));
            }
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float pp = pw[h][j];
                acc[h][0] += pp * c0;
                acc[h][1] += pp * c1;
            }
        }
        __syncthreads();
    }

#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float z = wave_sum(zl[h]);
        const float safe_l = l[h] > 0.f ? l[h] : 1.f;
        const float inv = 1.f / safe_l;
        float *row = mid_o + (((int64_t)b * num_q_heads + kvh * G + h) * num_splits + sid) *
                                 (kHeadDim + 1);
        row[2 * lane] = (acc[h][0] + z) * inv;
        row[2 * lane + 1] = (acc[h][1] + z) * inv;
        if (lane == 0)
            row[kHeadDim] = m[h] * kLn2 + logf(safe_l);
    }
}

}  // namespace tq4
