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
// the MFMA kernel and its cross-check on the GPU.
#pragma once
#include "tq4_device.h"

namespace tq4 {

// KF8: the FP8-key preset -- K is one E4M3 byte per dim (no codebook, no norm, the query
// is not rotated); record D + D/2 bytes (SoA; two metadata fields: V scale, V zero) or a
// D + D/2 + 4 byte slot (AoS: V scale and zero after the V codes).
template <int LAYOUT, int G, bool KF8 = false>
__global__ __launch_bounds__(kWave) void stage1_simple_kernel(
    const float *__restrict__ q_rot, const uint8_t *__restrict__ cache,
    const int32_t *__restrict__ block_table, const int32_t *__restrict__ seq_lens,
    const float *__restrict__ pair_lut, float *__restrict__ mid_o, const float *__restrict__ sinks,
    int num_q_heads, int num_kv_heads, int block_size, int max_blocks, int64_t block_stride,
    int num_splits, float score_scale_log2) {
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

    if (!KF8 && lane < 16)
        lut[lane] = pair_lut[2 * (lane * 16)];  // row (lane, 0) = (c[lane], c[0])
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

    for (int t0 = r.start; t0 < r.end; t0 += kWave) {
        const int t = t0 + lane;
        const bool valid = t < r.end;
        const int tc = valid ? t : r.end - 1;
        const int64_t blk = bt[tc / block_size];
        const int off = tc % block_size;
        const uint8_t *kp, *vp;
        float norm, vscale, vzero;
        if constexpr (KF8) {
            constexpr int rec = kHeadDim + kHalfD;
            if (LAYOUT == 0) {
                kp = cache + blk * block_stride + ((int64_t)off * num_kv_heads + kvh) * rec;
                const uint8_t *meta = cache + blk * block_stride + (int64_t)block_size * num_kv_heads * rec +
                                      ((int64_t)kvh * 2 * block_size + off) * 2;
                vscale = load_half(meta);
                vzero = load_half(meta + 2 * block_size);
            } else {
                kp = cache + blk * block_stride + ((int64_t)off * num_kv_heads + kvh) * (rec + 4);
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
            kp = aos_slot(cache, blk, block_stride, off, num_kv_heads, kvh);
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
        if constexpr (KF8) {
            for (int w = 0; w < kHeadDim / 4; ++w) {
                const uint32_t word = load_u32_a2(kp + 4 * w);
                const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)word, false);
                const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)word, true);
                const float k4[4] = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
                for (int n = 0; n < 4; ++n)
#pragma unroll
                    for (int h = 0; h < G; ++h)
                        s[h] += qs[h][4 * w + n] * k4[n];
            }
            for (int w = 0; w < kHalfD / 4; ++w)
                vstage[lane][w] = load_u32_a2(vp + 4 * w);
        } else {
            for (int w = 0; w < kHalfD / 4; ++w) {
                const uint32_t word = load_u32_a2(kp + 4 * w);
#pragma unroll
                for (int n = 0; n < 8; ++n) {
                    const float c = lut[(word >> (4 * n)) & 15u];
                    if (LAYOUT == 1)
                        csq += c * c;
#pragma unroll
                    for (int h = 0; h < G; ++h)
                        s[h] += qs[h][8 * w + n] * c;
                }
                vstage[lane][w] = load_u32_a2(vp + 4 * w);
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
            const uint32_t word = vstage[j][lane >> 2];
            const uint32_t byte = (word >> (8 * (lane & 3))) & 0xFFu;
            const float c0 = (float)(byte & 15u), c1 = (float)(byte >> 4);
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
