/*
 * Plain-C float32 restatement of the TurboQuant 4-bit decode Stage1 and Stage2.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ and by the cpu_baseline leg of
 * bench.py through oracle/native.py.  Nothing in the shipped package links it.
 *
 * tq4o_stage1 restates one Triton V1 Stage1 program per (batch, q-head, split)
 * exactly as the reference oracle kernels do it:
 *   - split partition + empty-split return ........ reference/soa_decode_v1.py:101-110
 *   - BLOCK_KV = 4 token steps (baseline/triton_v1.py:85)
 *   - SoA addressing ............................... reference/soa_decode_v1.py:156-188
 *   - AoS addressing ............................... reference/aos_decode.py:140-152
 *   - K: centroid gather, SoA folded norm .......... reference/soa_decode_v1.py:213-254
 *     AoS norm correction c / sqrt(sum c^2 + 1e-16) reference/aos_decode.py:199-224
 *   - online softmax (natural exp) ................. reference/soa_decode_v1.py:259-265
 *   - V: code * scale + zero ....................... reference/soa_decode_v1.py:285-300
 *   - acc / l update and epilogue (safe_l, m+ln l) . reference/soa_decode_v1.py:302-314
 * tq4o_stage2 restates baseline/stage2.py:26-55 (running merge over non-empty splits).
 *
 * Parity: cross-checked against the float64 numpy restatement (oracle/stage1.py),
 * which is itself checked against torch's attention routines.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define TQ4O_MAX_D 256
#define TQ4O_BLOCK_KV 4

static inline float tq4o_half_to_float(const uint8_t *p) {
    uint16_t h = (uint16_t)(p[0] | ((uint16_t)p[1] << 8));
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t expo = (h >> 10) & 0x1F;
    uint32_t mant = h & 0x3FF;
    uint32_t bits;
    if (expo == 0) {
        if (mant == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do {
                e++;
                mant <<= 1;
            } while ((mant & 0x400) == 0);
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((mant & 0x3FF) << 13);
        }
    } else if (expo == 31) {
        bits = sign | 0x7F800000u | (mant << 13);
    } else {
        bits = sign | ((expo + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* Decode one token of one kv-head: K (already norm-scaled) and V into k[], v[]. */
static void tq4o_decode_token(const uint8_t *cache, int64_t block, int off, int kvh, int Hk,
                              int D, int bs, int64_t block_stride, int is_aos,
                              const float *cents, float *k_unit, float *k_norm, float *v) {
    const int half = D / 2;
    const uint8_t *kb, *vb;
    float norm, scale, zero;
    if (is_aos) {
        const int slot = D + 6 + ((D + 6) & 1);
        const uint8_t *s = cache + block * block_stride + (int64_t)off * Hk * slot + (int64_t)kvh * slot;
        kb = s;
        vb = s + half + 2;
        norm = tq4o_half_to_float(s + half);
        scale = tq4o_half_to_float(s + D + 2);
        zero = tq4o_half_to_float(s + D + 4);
    } else {
        const uint8_t *blk = cache + block * block_stride;
        const uint8_t *d = blk + (int64_t)off * Hk * D + (int64_t)kvh * D;
        const uint8_t *meta = blk + (int64_t)bs * Hk * D;
        kb = d;
        vb = d + half;
        norm = tq4o_half_to_float(meta + ((kvh * 3 + 0) * bs + off) * 2);
        scale = tq4o_half_to_float(meta + ((kvh * 3 + 1) * bs + off) * 2);
        zero = tq4o_half_to_float(meta + ((kvh * 3 + 2) * bs + off) * 2);
    }
    for (int j = 0; j < half; ++j) {
        k_unit[2 * j] = cents[kb[j] & 0xF];
        k_unit[2 * j + 1] = cents[kb[j] >> 4];
        v[2 * j] = (float)(vb[j] & 0xF) * scale + zero;
        v[2 * j + 1] = (float)(vb[j] >> 4) * scale + zero;
    }
    if (is_aos) {
        float sq = 0.0f;
        for (int d = 0; d < D; ++d)
            sq += k_unit[d] * k_unit[d];
        const float inv = 1.0f / sqrtf(sq + 1e-16f);
        for (int d = 0; d < D; ++d)
            k_unit[d] = k_unit[d] * inv;
    }
    *k_norm = norm;
}

int tq4o_stage1(const float *q_rot, const uint8_t *cache, const int32_t *block_table,
                const int32_t *seq_lens, const float *cents, float *mid_o, int B, int Hq,
                int Hk, int D, int bs, int max_blocks, int64_t block_stride, int S,
                int is_aos, float attn_scale, int nthreads) {
    if (D > TQ4O_MAX_D || D % 2 || Hq % Hk || bs <= 0 || S <= 0)
        return 1;
    const int G = Hq / Hk;
    const int64_t programs = (int64_t)B * Hq * S;
#ifdef _OPENMP
    if (nthreads > 0)
        omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 16)
#endif
    for (int64_t pid = 0; pid < programs; ++pid) {
        const int sid = (int)(pid % S);
        const int h = (int)((pid / S) % Hq);
        const int b = (int)(pid / ((int64_t)S * Hq));
        const int kvh = h / G;
        const int seq_len = seq_lens[b];
        const int split_len = (seq_len + S - 1) / S;
        const int start = split_len * sid;
        const int end = start + split_len < seq_len ? start + split_len : seq_len;
        if (start >= end)
            continue;
        const float *q = q_rot + ((int64_t)b * Hq + h) * D;
        float acc[TQ4O_MAX_D], k[TQ4O_MAX_D], v[TQ4O_BLOCK_KV][TQ4O_MAX_D];
        float m = -INFINITY, l = 0.0f;
        for (int d = 0; d < D; ++d)
            acc[d] = 0.0f;
        for (int t0 = start; t0 < end; t0 += TQ4O_BLOCK_KV) {
            float s[TQ4O_BLOCK_KV];
            float tile_max = -INFINITY;
            for (int j = 0; j < TQ4O_BLOCK_KV; ++j) {
                const int t = t0 + j;
                if (t >= end) {
                    s[j] = -INFINITY;
                    for (int d = 0; d < D; ++d)
                        v[j][d] = 0.0f;
                    continue;
                }
                const int64_t block = block_table[(int64_t)b * max_blocks + t / bs];
                float norm;
                tq4o_decode_token(cache, block, t % bs, kvh, Hk, D, bs, block_stride, is_aos,
                                  cents, k, &norm, v[j]);
                float term = 0.0f;
                for (int d = 0; d < D; ++d)
                    term += q[d] * k[d];
                s[j] = norm * term * attn_scale;
                if (s[j] > tile_max)
                    tile_max = s[j];
            }
            const float n_max = tile_max > m ? tile_max : m;
            const float re_scale = expf(m - n_max);
            float p[TQ4O_BLOCK_KV], psum = 0.0f;
            for (int j = 0; j < TQ4O_BLOCK_KV; ++j) {
                p[j] = expf(s[j] - n_max);
                psum += p[j];
            }
            for (int d = 0; d < D; ++d) {
                float pv = 0.0f;
                for (int j = 0; j < TQ4O_BLOCK_KV; ++j)
                    pv += p[j] * v[j][d];
                acc[d] = acc[d] * re_scale + pv;
            }
            l = l * re_scale + psum;
            m = n_max;
        }
        float *out = mid_o + (((int64_t)b * Hq + h) * S + sid) * (D + 1);
        const float safe_l = l > 0.0f ? l : 1.0f;
        for (int d = 0; d < D; ++d)
            out[d] = acc[d] / safe_l;
        out[D] = m + logf(safe_l);
    }
    return 0;
}

int tq4o_stage2(const float *mid_o, const int32_t *seq_lens, float *out, float *lse, int B,
                int Hq, int D, int S, int nthreads) {
    if (D > TQ4O_MAX_D || S <= 0)
        return 1;
#ifdef _OPENMP
    if (nthreads > 0)
        omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
#endif
    for (int64_t bh = 0; bh < (int64_t)B * Hq; ++bh) {
        const int b = (int)(bh / Hq);
        const int seq_len = seq_lens[b];
        const int split_len = (seq_len + S - 1) / S;
        float acc[TQ4O_MAX_D];
        for (int d = 0; d < D; ++d)
            acc[d] = 0.0f;
        float run_max = -INFINITY, run_sum = 0.0f;
        const float *base = mid_o + bh * (int64_t)S * (D + 1);
        for (int sid = 0; sid < S; ++sid) {
            const int start = split_len * sid;
            const int end = start + split_len < seq_len ? start + split_len : seq_len;
            if (end <= start)
                continue;
            const float *row = base + (int64_t)sid * (D + 1);
            const float split_lse = row[D];
            const float new_max = run_max > split_lse ? run_max : split_lse;
            const float old_scale = expf(run_max - new_max);
            const float weight = expf(split_lse - new_max);
            for (int d = 0; d < D; ++d)
                acc[d] = acc[d] * old_scale + weight * row[d];
            run_sum = run_sum * old_scale + weight;
            run_max = new_max;
        }
        for (int d = 0; d < D; ++d)
            out[bh * D + d] = acc[d] / run_sum;
        lse[bh] = run_max + logf(run_sum);
    }
    return 0;
}

int tq4o_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
