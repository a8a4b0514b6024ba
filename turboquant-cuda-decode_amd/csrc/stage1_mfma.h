// Stage1, matrix-core kernel (gfx950): one wave64 per (split, kv-head, sequence),
// GQA group G = 4 * NSET, 16-token tiles aligned to the KV block.
//
// Both products run on v_mfma_f32_4x4x1f32 (16 independent 4x4 outer-product blocks,
// exact fp32 operands, fp32 accumulate).  Lane l = 16u + 4v + c  (u, v, c in 0..3);
// MFMA block = l / 4 = 4u + v, in-block index = c.
//
// QK^T of a tile (tokens 4u + i, i = 0..3):
//   A[block][row i] = K[4u + i][32v + s]      lane (u,v,c) decodes token 4u + c,
//   B[block][col j] = q[head j][32v + s]      dims 32v .. 32v+31 (16 code bytes,
//   32 steps s; result lane (u,v,j) reg i     one 16-byte load), q held in VGPRs.
//   = partial dot over dim group v.  Two DPP row rotations (ror 8, ror 4) sum the four
//   dim groups, leaving the full score of token 4u + i, head c in every lane (u,*,c).
// Softmax: each lane keeps the running (m, l, z) of its slot u and head c.  All four
//   lanes (u, 0..3, c) hold identical scores, so their states agree.  The running max
//   only moves when a score exceeds it by more than kRescaleLog2 (p <= 2^8), so the
//   32-register rescale is rare after the first tile; slots merge once at the end.
// PV of the tile, step i (token 4u + i), 8 MFMAs k = 0..7:
//   A[block][row r] = code[4u + i][32v + 8r + k]   lane (u,v,c) loads one V dword
//   B[block][col j] = p[head j][4u + i] * scale    (its own softmax weight)
//   result lane (u,v,j) reg r += O[head j][32v + 8r + k]   (32 accumulators / set)
//   The V zero term sum_t p_t * zero_t is kept per lane and added at the end.
#pragma once
#include "tq4_device.h"

namespace tq4 {

constexpr float kRescaleLog2 = 8.0f;

template <int CTRL> __device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
// Sum over the four lanes of a 16-lane row that share (lane & 3).
__device__ __forceinline__ float row_group_sum(float x) {
    x += dpp<0x128>(x);  // row_ror:8
    x += dpp<0x124>(x);  // row_ror:4
    return x;
}
// Value of quad lane Q broadcast to the whole quad.
template <int Q> __device__ __forceinline__ float quad_bcast(float x) {
    return dpp<(Q | (Q << 2) | (Q << 4) | (Q << 6))>(x);
}

__device__ __forceinline__ floatx4 mfma4x4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 0);
}

template <int LAYOUT, int NSET>
__global__ __launch_bounds__(kWave) void stage1_mfma_kernel(
    const float *__restrict__ q_rot, const uint8_t *__restrict__ cache,
    const int32_t *__restrict__ block_table, const int32_t *__restrict__ seq_lens,
    const float *__restrict__ pair_lut, float *__restrict__ mid_o, int num_q_heads,
    int num_kv_heads, int block_size, int max_blocks, int64_t block_stride, int num_splits,
    float score_scale_log2) {
    constexpr int G = 4 * NSET;
    const int sid = blockIdx.x;
    const int kvh = blockIdx.y;
    const int b = blockIdx.z;
    const int lane = threadIdx.x;
    const SplitRange rng = split_range(seq_lens[b], num_splits, sid);
    if (rng.start >= rng.end)
        return;
    const int c = lane & 3;
    const int v = (lane >> 2) & 3;
    const int u = lane >> 4;

    __shared__ float lut[16];
    if (lane < 16)
        lut[lane] = pair_lut[32 * lane];  // row (lane, 0) = (c[lane], c[0])

    float qreg[NSET][32];
#pragma unroll
    for (int set = 0; set < NSET; ++set) {
        const float4 *qp = reinterpret_cast<const float4 *>(
            q_rot + ((int64_t)b * num_q_heads + kvh * G + 4 * set + c) * kHeadDim + 32 * v);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float4 x = qp[j];
            qreg[set][4 * j + 0] = x.x;
            qreg[set][4 * j + 1] = x.y;
            qreg[set][4 * j + 2] = x.z;
            qreg[set][4 * j + 3] = x.w;
        }
    }

    float m[NSET], l[NSET], z[NSET];
    floatx4 acc[NSET][8];
#pragma unroll
    for (int set = 0; set < NSET; ++set) {
        m[set] = -INFINITY;
        l[set] = 0.f;
        z[set] = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            acc[set][k] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    __syncthreads();

    const int32_t *bt = block_table + (int64_t)b * max_blocks;
    const int tile_first = rng.start & ~15;
    const int tile_last = (rng.end - 1) & ~15;

    for (int t0 = tile_first; t0 <= tile_last; t0 += 16) {
        const int64_t blk = bt[t0 / block_size];
        const int toff = t0 % block_size;

        // ---- loads: K (own token 4u + c), V (tokens 4u + i), metadata (tokens 4u + i)
        uint32_t kw[4], vw[4];
        float norm[4], vscale[4], vzero[4];
        float csq_part = 0.f;
        if (LAYOUT == 0) {
            const uint8_t *rec = soa_record(cache, blk, block_stride, toff + 4 * u + c,
                                            num_kv_heads, kvh);
            const uint4 kq = *reinterpret_cast<const uint4 *>(rec + 16 * v);
            kw[0] = kq.x;
            kw[1] = kq.y;
            kw[2] = kq.z;
            kw[3] = kq.w;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint8_t *ri = soa_record(cache, blk, block_stride, toff + 4 * u + i,
                                               num_kv_heads, kvh);
                vw[i] = *reinterpret_cast<const uint32_t *>(ri + kHalfD + 16 * v + 4 * c);
            }
            const uint2 nq = *reinterpret_cast<const uint2 *>(
                soa_meta(cache, blk, block_stride, toff + 4 * u, num_kv_heads, kvh, block_size, 0));
            const uint2 sq = *reinterpret_cast<const uint2 *>(
                soa_meta(cache, blk, block_stride, toff + 4 * u, num_kv_heads, kvh, block_size, 1));
            const uint2 zq = *reinterpret_cast<const uint2 *>(
                soa_meta(cache, blk, block_stride, toff + 4 * u, num_kv_heads, kvh, block_size, 2));
            norm[0] = half_bits_to_float(nq.x);
            norm[1] = half_bits_to_float(nq.x >> 16);
            norm[2] = half_bits_to_float(nq.y);
            norm[3] = half_bits_to_float(nq.y >> 16);
            vscale[0] = half_bits_to_float(sq.x);
            vscale[1] = half_bits_to_float(sq.x >> 16);
            vscale[2] = half_bits_to_float(sq.y);
            vscale[3] = half_bits_to_float(sq.y >> 16);
            vzero[0] = half_bits_to_float(zq.x);
            vzero[1] = half_bits_to_float(zq.x >> 16);
            vzero[2] = half_bits_to_float(zq.y);
            vzero[3] = half_bits_to_float(zq.y >> 16);
        } else {
            const uint8_t *slot = aos_slot(cache, blk, block_stride, toff + 4 * u + c,
                                           num_kv_heads, kvh);
            const uint8_t *kb = slot + 16 * v;
            const uint32_t *ka = reinterpret_cast<const uint32_t *>(
                reinterpret_cast<uintptr_t>(kb) & ~uintptr_t(3));
            const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(kb) & 3);
            uint32_t a5[5];
#pragma unroll
            for (int j = 0; j < 5; ++j)
                a5[j] = ka[j];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                kw[j] = __builtin_amdgcn_alignbyte(a5[j + 1], a5[j], sh);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint8_t *vb = aos_slot(cache, blk, block_stride, toff + 4 * u + i,
                                             num_kv_heads, kvh) + kHalfD + 2 + 16 * v + 4 * c;
                const uint32_t *va = reinterpret_cast<const uint32_t *>(
                    reinterpret_cast<uintptr_t>(vb) & ~uintptr_t(3));
                vw[i] = __builtin_amdgcn_alignbyte(va[1], va[0],
                                                   (uint32_t)(reinterpret_cast<uintptr_t>(vb) & 3));
            }
            const float own_norm = load_half(slot + kHalfD);
            const float own_scale = load_half(slot + kHeadDim + 2);
            const float own_zero = load_half(slot + kHeadDim + 4);
            norm[0] = quad_bcast<0>(own_norm);
            norm[1] = quad_bcast<1>(own_norm);
            norm[2] = quad_bcast<2>(own_norm);
            norm[3] = quad_bcast<3>(own_norm);
            vscale[0] = quad_bcast<0>(own_scale);
            vscale[1] = quad_bcast<1>(own_scale);
            vscale[2] = quad_bcast<2>(own_scale);
            vscale[3] = quad_bcast<3>(own_scale);
            vzero[0] = quad_bcast<0>(own_zero);
            vzero[1] = quad_bcast<1>(own_zero);
            vzero[2] = quad_bcast<2>(own_zero);
            vzero[3] = quad_bcast<3>(own_zero);
        }

        // ---- QK^T on the matrix cores
        floatx4 sc[NSET];
#pragma unroll
        for (int set = 0; set < NSET; ++set)
            sc[set] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int n = 0; n < 8; ++n) {
                const float kv = lut[(kw[j] >> (4 * n)) & 15u];
                if (LAYOUT == 1)
                    csq_part += kv * kv;
#pragma unroll
                for (int set = 0; set < NSET; ++set)
                    sc[set] = mfma4x4(kv, qreg[set][8 * j + n], sc[set]);
            }
        }

        float kscale[4];
        if (LAYOUT == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                kscale[i] = norm[i];
        } else {
            const float csq = row_group_sum(csq_part);  // ||c[idx]||^2 of token 4u + c
            const float inv_own = 1.0f / sqrtf(csq + 1e-16f);
            kscale[0] = norm[0] * quad_bcast<0>(inv_own);
            kscale[1] = norm[1] * quad_bcast<1>(inv_own);
            kscale[2] = norm[2] * quad_bcast<2>(inv_own);
            kscale[3] = norm[3] * quad_bcast<3>(inv_own);
        }

        bool valid[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tok = t0 + 4 * u + i;
            valid[i] = tok >= rng.start && tok < rng.end;
        }

        // ---- per-slot online softmax (exp2 domain) and PV weights
        float pw[NSET][4];
#pragma unroll
        for (int set = 0; set < NSET; ++set) {
            float s2[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float dot = row_group_sum(sc[set][i]);
                s2[i] = valid[i] ? dot * kscale[i] * score_scale_log2 : -INFINITY;
            }
            const float tmax = fmaxf(fmaxf(s2[0], s2[1]), fmaxf(s2[2], s2[3]));
            const bool need = tmax > m[set] + kRescaleLog2;
            if (__any(need)) {
                const float mnew = need ? tmax : m[set];
                const float alpha = need ? exp2f(m[set] - mnew) : 1.f;
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    acc[set][k] *= alpha;
                l[set] *= alpha;
                z[set] *= alpha;
                m[set] = mnew;
            }
            const float m_eff = m[set] == -INFINITY ? 0.f : m[set];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float p = exp2f(s2[i] - m_eff);
                l[set] += p;
                z[set] += valid[i] ? p * vzero[i] : 0.f;
                pw[set][i] = valid[i] ? p * vscale[i] : 0.f;
            }
        }

        // ---- PV on the matrix cores
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = vw[i] & 0x0F0F0F0Fu;
            const uint32_t hi = (vw[i] >> 4) & 0x0F0F0F0Fu;
            float cv[8];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                cv[2 * q] = (float)((lo >> (8 * q)) & 0xFFu);
                cv[2 * q + 1] = (float)((hi >> (8 * q)) & 0xFFu);
            }
#pragma unroll
            for (int k = 0; k < 8; ++k)
#pragma unroll
                for (int set = 0; set < NSET; ++set)
                    acc[set][k] = mfma4x4(cv[k], pw[set][i], acc[set][k]);
        }
    }

    // ---- merge the four slots u and write this split's rows
#pragma unroll
    for (int set = 0; set < NSET; ++set) {
        float mx = fmaxf(m[set], __shfl_xor(m[set], 16, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        const float f = m[set] == -INFINITY ? 0.f : exp2f(m[set] - mx);
        float lt = f * l[set];
        lt += __shfl_xor(lt, 16, kWave);
        lt += __shfl_xor(lt, 32, kWave);
        const float zf = f * z[set];
        const float safe_l = lt > 0.f ? lt : 1.f;
        const float inv = 1.f / safe_l;
        float *row = mid_o + (((int64_t)b * num_q_heads + kvh * G + 4 * set + c) * num_splits + sid) *
                                 (kHeadDim + 1);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float o = f * acc[set][k][r] + zf;
                o += __shfl_xor(o, 16, kWave);
                o += __shfl_xor(o, 32, kWave);
                if (r == u)
                    row[32 * v + 8 * r + k] = o * inv;
            }
        }
        if (lane < 4)
            row[kHeadDim] = mx * kLn2 + logf(safe_l);
    }
}

}  // namespace tq4
