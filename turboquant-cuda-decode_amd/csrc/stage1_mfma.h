// Stage1, matrix-core kernel (gfx950): one wave64 per (split, kv-head, sequence),
// GQA group G = 4 * NSET, 16-token tiles aligned to the KV block.
//
// Lane l = 16u + 4v + c (u, v, c in 0..3).  MFMA block = l / 4 = 4u + v, in-block
// index = c.  The 4x4 MFMA shapes put 4 tokens (or 4 dims) on the rows and the 4
// heads of a head set on the columns, so the GQA group costs no padding.
//
// QK^T of a tile (tokens 4u + i, i = 0..3) on v_mfma_f32_4x4x1f32 (fp32 operands):
//   A[block][row i] = K[4u + i][32v + s]      lane (u,v,c) decodes token 4u + c,
//   B[block][col j] = q[head j][32v + s]      dims 32v .. 32v+31 (16 code bytes,
//   32 steps s; result lane (u,v,j) reg i     one 16-byte load).
//   B needs the same value in the four lane groups u, so it is broadcast from lane
//   group s % 4 by the MFMA's B lane-group pattern (blgp = 4 + s % 4): lane (g,v,c)
//   holds q[c][32v + 4k + g] in register k, 8 registers per head set.
//   = partial dot over dim group v.  The centroids come from a 256-entry LDS table
//   indexed by the packed code byte (entry = (c[low nibble], c[high nibble])): one
//   ds_read_b64 per byte gives the A operands of two MFMAs.  q is pre-scaled by
//   attn_scale * log2(e).  Two DPP row rotations (ror 8, ror 4) sum the four dim
//   groups, leaving the score of token 4u + i, head c in every lane (u,*,c).
// Softmax: each lane keeps the running (m, l, z) of its slot u and head c.  All four
//   lanes (u, 0..3, c) hold identical scores, so their states agree.  The running max
//   only moves when a score exceeds it by more than kRescaleLog2 (p <= 2^8), so the
//   32-register rescale is rare after the first tile; slots merge once at the end.
// PV of the tile on v_mfma_f32_4x4x1f32 (fp32 operands), step i (token 4u + i), 8
//   MFMAs k = 0..7:
//   A[block][row r] = code[4u + i][32v + 8r + k]   lane (u,v,c) loads one V dword
//   B[block][col j] = p[head j][4u + i] * scale    (its own softmax weight)
//   result lane (u,v,j) reg r += O[head j][32v + 8r + k]   (32 accumulators / set)
//   The V zero term sum_t p_t * zero_t is kept per lane and added at the end.
//
// Schedule: stage j = softmax of tile j, then PV of tile j together with QK^T of tile
// j+1 in one branch-free block (software pipelining across tiles), so matrix-core and
// vector work from two tiles overlap within a wave.
//
// Memory: the block-table entries of up to 64 tiles are read once (one lane per tile)
// and broadcast with readlane.  A 4-slot register ring keeps the loads of the next
// tiles in flight (~6.6-8.8 KB per wave).  Loads are buffer loads off a per-tile
// descriptor whose base is the KV block (offsets are per-lane constants), plain and
// unconditional, so the compiler's wait before each tile is exact.
#pragma once
#include "tq4_device.h"

namespace tq4 {

constexpr float kRescaleLog2 = 8.0f;


template <int CTRL> __device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
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

__device__ __forceinline__ floatx4 mfma_f32(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 0);
}
// Same, with B taken from lane group G (lanes 16G .. 16G+15) for all four groups.
template <int G> __device__ __forceinline__ floatx4 mfma_f32_bcast(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 4 + G);
}

// Hide a value's provenance from the optimiser so byte-wise decodes stay single
// instructions (v_cvt_f32_ubyteN) instead of being re-derived with extra shifts.
__device__ __forceinline__ uint32_t opaque(uint32_t x) {
    __asm__("" : "+v"(x));
    return x;
}

// K-code table entry for one packed byte (low nibble = even dim, high nibble = odd
// dim): SoA (c[lo], c[hi]); AoS adds c[lo]^2 + c[hi]^2 for the norm correction.
template <int LAYOUT> struct KEntry;
template <> struct KEntry<0> { typedef float2 type; };
template <> struct KEntry<1> { typedef float4 type; };

template <int LAYOUT>
__device__ __forceinline__ void build_key_table(typename KEntry<LAYOUT>::type *tbl,
                                                const float *pair_lut, int lane) {
    for (int e = lane; e < 256; e += kWave) {
        const int lo = e & 15, hi = e >> 4;
        const float c_lo = pair_lut[2 * (lo * 16 + hi)];      // row (lo, hi) = (c[lo], c[hi])
        const float c_hi = pair_lut[2 * (lo * 16 + hi) + 1];
        if constexpr (LAYOUT == 0)
            tbl[e] = make_float2(c_lo, c_hi);
        else
            tbl[e] = make_float4(c_lo, c_hi, c_lo * c_lo + c_hi * c_hi, 0.f);
    }
}

// Registers one tile needs (decoded view).
struct TileRegs {
    uint4 k;       // own token's 16 K code bytes (dims 32v .. 32v+31)
    uint32_t v[4]; // V code dword of token 4u + i (dims 32v + 8c .. +7)
    uint2 m[3];    // SoA: fp16 norm / scale / zero of tokens 4u .. 4u+3
                   // AoS: m[0].x = own norm, m[0].y = own scale, m[1].x = own zero
};

// Per-lane byte offsets inside one KV block (fixed for a kernel instance).
struct LaneOffsets {
    uint32_t k, v[4], m, mf;  // mf: SoA distance between the three metadata arrays
};

template <int LAYOUT>
__device__ __forceinline__ LaneOffsets lane_offsets(int u, int v, int c, int kvh, int hk,
                                                    int block_size) {
    LaneOffsets o;
    if (LAYOUT == 0) {
        o.k = ((4 * u + c) * hk + kvh) * kSoaRecord + 16 * v;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            o.v[i] = ((4 * u + i) * hk + kvh) * kSoaRecord + kHalfD + 16 * v + 4 * c;
        o.m = block_size * hk * kSoaRecord + (kvh * 3 * block_size + 4 * u) * 2;
        o.mf = block_size * 2;
    } else {
        o.k = ((4 * u + c) * hk + kvh) * kAosSlot + 16 * v;  // 2-byte aligned
#pragma unroll
        for (int i = 0; i < 4; ++i)
            o.v[i] = ((4 * u + i) * hk + kvh) * kAosSlot + kHalfD + 2 + 16 * v + 4 * c;
        o.m = ((4 * u + c) * hk + kvh) * kAosSlot;  // own slot start
        o.mf = 0;
    }
    return o;
}

// Raw loads of one tile (plain loads, so the compiler tracks their completion).
template <int LAYOUT> struct RawTile;
template <> struct RawTile<0> {
    uint4 k;
    uint32_t v[4];
    uint2 m[3];
};
template <> struct RawTile<1> {
    uint32_t k[5];  // aligned dwords around the own (2-byte aligned) K bytes
    uint2 v[4];     // aligned dword pairs around each V dword
    unsigned short norm, scale, zero;
};

// Loads of one tile.  rsrc: buffer descriptor based at the KV block; doff / moff: byte
// offsets of the tile's 16-token piece inside the block (data records / SoA metadata).
// Offsets are the per-lane constants of lane_offsets().
template <int LAYOUT>
__device__ __forceinline__ void issue_tile(RawTile<LAYOUT> &t, __amdgpu_buffer_rsrc_t rsrc,
                                           int doff, int moff, const LaneOffsets &o) {
    if constexpr (LAYOUT == 0) {
        t.k = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, o.k, doff, 0));
#pragma unroll
        for (int i = 0; i < 4; ++i)
            t.v[i] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, o.v[i], doff, 0);
#pragma unroll
        for (int f = 0; f < 3; ++f)
            t.m[f] = __builtin_bit_cast(
                uint2, __builtin_amdgcn_raw_buffer_load_b64(rsrc, o.m + f * o.mf, moff, 0));
    } else {
        const uint32_t ka = o.k & ~3u;
        const auto k03 = __builtin_amdgcn_raw_buffer_load_b128(rsrc, ka, doff, 0);
        t.k[0] = k03[0];
        t.k[1] = k03[1];
        t.k[2] = k03[2];
        t.k[3] = k03[3];
        t.k[4] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, ka + 16, doff, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            t.v[i] = __builtin_bit_cast(
                uint2, __builtin_amdgcn_raw_buffer_load_b64(rsrc, o.v[i] & ~3u, doff, 0));
        t.norm = __builtin_amdgcn_raw_buffer_load_b16(rsrc, o.m + kHalfD, doff, 0);
        t.scale = __builtin_amdgcn_raw_buffer_load_b16(rsrc, o.m + kHeadDim + 2, doff, 0);
        t.zero = __builtin_amdgcn_raw_buffer_load_b16(rsrc, o.m + kHeadDim + 4, doff, 0);
    }
}

// Decoded view of a tile's registers (AoS dwords funnel-shifted into place).
template <int LAYOUT>
__device__ __forceinline__ TileRegs decode_tile(const RawTile<LAYOUT> &t, const LaneOffsets &o) {
    TileRegs r;
    if constexpr (LAYOUT == 0) {
        r.k = t.k;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            r.v[i] = t.v[i];
#pragma unroll
        for (int f = 0; f < 3; ++f)
            r.m[f] = t.m[f];
    } else {
        const uint32_t sh = o.k & 3u;
        r.k.x = __builtin_amdgcn_alignbyte(t.k[1], t.k[0], sh);
        r.k.y = __builtin_amdgcn_alignbyte(t.k[2], t.k[1], sh);
        r.k.z = __builtin_amdgcn_alignbyte(t.k[3], t.k[2], sh);
        r.k.w = __builtin_amdgcn_alignbyte(t.k[4], t.k[3], sh);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            r.v[i] = __builtin_amdgcn_alignbyte(t.v[i].y, t.v[i].x, o.v[i] & 3u);
        r.m[0] = uint2{t.norm, t.scale};
        r.m[1] = uint2{t.zero, 0u};
        r.m[2] = uint2{0u, 0u};
    }
    return r;
}

template <int NSET> struct SoftmaxState {
    float m[NSET], l[NSET], z[NSET];
    floatx4 acc[NSET][8];
};

// q in the exp2 domain: lane (g,v,c) holds q[head 4*set + c][32v + 4k + g] in v[set][k].
template <int NSET> struct QOperands {
    float v[NSET][8];
};

__device__ __forceinline__ float half_lo(uint32_t w) { return half_bits_to_float(w); }
__device__ __forceinline__ float half_hi(uint32_t w) { return half_bits_to_float(w >> 16); }

// Partial QK^T dots of one tile (two accumulation chains per head set) and, for AoS,
// the lane's share of ||c[idx]||^2 of its own token.
template <int NSET> struct TileScores {
    floatx4 sc0[NSET], sc1[NSET];
    float csq_part;
};

template <int LAYOUT, int NSET>
__device__ __forceinline__ void qk_tile(const uint4 &k, const typename KEntry<LAYOUT>::type *ktab,
                                        const QOperands<NSET> &q, TileScores<NSET> &s) {
#pragma unroll
    for (int set = 0; set < NSET; ++set) {
        s.sc0[set] = floatx4{0.f, 0.f, 0.f, 0.f};
        s.sc1[set] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    s.csq_part = 0.f;
    const uint32_t kwords[4] = {k.x, k.y, k.z, k.w};
#pragma unroll
    for (int bidx = 0; bidx < 16; ++bidx) {
        const auto e = ktab[(kwords[bidx >> 2] >> (8 * (bidx & 3))) & 0xFFu];  // dims 2b, 2b+1
        if constexpr (LAYOUT == 1)
            s.csq_part += e.z;
#pragma unroll
        for (int set = 0; set < NSET; ++set) {
            // dims 2b and 2b+1 = 4k + g with k = b / 2, g = 2 (b % 2) + {0, 1}
            if (bidx & 1) {
                s.sc0[set] = mfma_f32_bcast<2>(e.x, q.v[set][bidx >> 1], s.sc0[set]);
                s.sc1[set] = mfma_f32_bcast<3>(e.y, q.v[set][bidx >> 1], s.sc1[set]);
            } else {
                s.sc0[set] = mfma_f32_bcast<0>(e.x, q.v[set][bidx >> 1], s.sc0[set]);
                s.sc1[set] = mfma_f32_bcast<1>(e.y, q.v[set][bidx >> 1], s.sc1[set]);
            }
        }
    }
}

// Scores of one tile -> per-slot online softmax update -> PV weights pw (p * V scale).
// MASKED selects the path for a tile that straddles the split boundary (tokens outside
// [start, end) get p = 0).
template <int LAYOUT, int NSET, bool MASKED>
__device__ __forceinline__ void softmax_tile(const TileScores<NSET> &s, const TileRegs &t,
                                             SoftmaxState<NSET> &st, float (&pw)[NSET][4],
                                             int tok0, int start, int end) {
    // per-token factors: K norm (score is already in the exp2 domain), V scale/zero
    float norm[4], vscale[4], vzero[4];
    if constexpr (LAYOUT == 0) {
        norm[0] = half_lo(t.m[0].x);
        norm[1] = half_hi(t.m[0].x);
        norm[2] = half_lo(t.m[0].y);
        norm[3] = half_hi(t.m[0].y);
        vscale[0] = half_lo(t.m[1].x);
        vscale[1] = half_hi(t.m[1].x);
        vscale[2] = half_lo(t.m[1].y);
        vscale[3] = half_hi(t.m[1].y);
        vzero[0] = half_lo(t.m[2].x);
        vzero[1] = half_hi(t.m[2].x);
        vzero[2] = half_lo(t.m[2].y);
        vzero[3] = half_hi(t.m[2].y);
    } else {
        const float csq = row_group_sum(s.csq_part);  // ||c[idx]||^2 of token 4u + c
        const float own_ks = half_lo(t.m[0].x) * (1.0f / sqrtf(csq + 1e-16f));
        const float own_scale = half_lo(t.m[0].y);
        const float own_zero = half_lo(t.m[1].x);
        norm[0] = quad_bcast<0>(own_ks);
        norm[1] = quad_bcast<1>(own_ks);
        norm[2] = quad_bcast<2>(own_ks);
        norm[3] = quad_bcast<3>(own_ks);
        vscale[0] = quad_bcast<0>(own_scale);
        vscale[1] = quad_bcast<1>(own_scale);
        vscale[2] = quad_bcast<2>(own_scale);
        vscale[3] = quad_bcast<3>(own_scale);
        vzero[0] = quad_bcast<0>(own_zero);
        vzero[1] = quad_bcast<1>(own_zero);
        vzero[2] = quad_bcast<2>(own_zero);
        vzero[3] = quad_bcast<3>(own_zero);
    }
    bool valid[4] = {true, true, true, true};
    if (MASKED) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            valid[i] = tok0 + i >= start && tok0 + i < end;
    }
#pragma unroll
    for (int set = 0; set < NSET; ++set) {
        float s2[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float dot = row_group_sum(s.sc0[set][i] + s.sc1[set][i]);
            s2[i] = dot * norm[i];
            if (MASKED)
                s2[i] = valid[i] ? s2[i] : -INFINITY;
        }
        const float tmax = fmaxf(fmaxf(s2[0], s2[1]), fmaxf(s2[2], s2[3]));
        const bool need = tmax > st.m[set] + kRescaleLog2;
        if (__any(need)) {
            const float mnew = need ? tmax : st.m[set];
            const float alpha = need ? __builtin_amdgcn_exp2f(st.m[set] - mnew) : 1.f;
#pragma unroll
            for (int k = 0; k < 8; ++k)
                st.acc[set][k] *= alpha;
            st.l[set] *= alpha;
            st.z[set] *= alpha;
            st.m[set] = mnew;
        }
        const float m_eff = MASKED && st.m[set] == -INFINITY ? 0.f : st.m[set];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float p = __builtin_amdgcn_exp2f(s2[i] - m_eff);
            st.l[set] += p;
            if (MASKED) {
                st.z[set] += valid[i] ? p * vzero[i] : 0.f;
                pw[set][i] = valid[i] ? p * vscale[i] : 0.f;
            } else {
                st.z[set] = fmaf(p, vzero[i], st.z[set]);
                pw[set][i] = p * vscale[i];
            }
        }
    }
}

// PV of one tile on the matrix cores (fp32 operands).
template <int NSET>
__device__ __forceinline__ void pv_tile(const TileRegs &t, const float (&pw)[NSET][4],
                                        SoftmaxState<NSET> &st) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = opaque(t.v[i] & 0x0F0F0F0Fu);
        const uint32_t hi = opaque((t.v[i] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            const float c0 = (float)((lo >> (8 * qq)) & 0xFFu);
            const float c1 = (float)((hi >> (8 * qq)) & 0xFFu);
#pragma unroll
            for (int set = 0; set < NSET; ++set) {
                st.acc[set][2 * qq] = mfma_f32(c0, pw[set][i], st.acc[set][2 * qq]);
                st.acc[set][2 * qq + 1] = mfma_f32(c1, pw[set][i], st.acc[set][2 * qq + 1]);
            }
        }
    }
}

template <int LAYOUT, int NSET>
__global__ __launch_bounds__(kWave) void stage1_mfma_kernel(
    const float *__restrict__ q_rot, const uint8_t *__restrict__ cache,
    const int32_t *__restrict__ block_table, const int32_t *__restrict__ seq_lens,
    const float *__restrict__ pair_lut, float *__restrict__ mid_o, int num_q_heads,
    int num_kv_heads, int block_size_log2, int max_blocks, int64_t block_stride, int num_splits,
    float score_scale_log2) {
    constexpr int G = 4 * NSET;
    const int block_size = 1 << block_size_log2;
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

    __shared__ typename KEntry<LAYOUT>::type ktab[256];
    build_key_table<LAYOUT>(ktab, pair_lut, lane);

    // q of heads (kvh*G + 4*set + c), dims 32v + 4k + u, scaled to the exp2 domain
    QOperands<NSET> q;
#pragma unroll
    for (int set = 0; set < NSET; ++set) {
        const float *qp =
            q_rot + ((int64_t)b * num_q_heads + kvh * G + 4 * set + c) * kHeadDim + 32 * v + u;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            q.v[set][k] = qp[4 * k] * score_scale_log2;
    }

    SoftmaxState<NSET> st;
#pragma unroll
    for (int set = 0; set < NSET; ++set) {
        st.m[set] = -INFINITY;
        st.l[set] = 0.f;
        st.z[set] = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            st.acc[set][k] = floatx4{0.f, 0.f, 0.f, 0.f};
    }

    const LaneOffsets off = lane_offsets<LAYOUT>(u, v, c, kvh, num_kv_heads, block_size);
    const int32_t *bt = block_table + (int64_t)b * max_blocks;
    const int tile_first = rng.start & ~15;
    const int ntiles = (((rng.end - 1) & ~15) - tile_first) / 16 + 1;
    __syncthreads();

    // Issue the loads of tile j (global index) into ring slot r; its block id sits in
    // lane (j mod 64) of bt_lane_val.
    auto issue = [&](RawTile<LAYOUT> &r, int bt_lane_val, int j) {
        const int blk = __builtin_amdgcn_readlane(bt_lane_val, j & 63);
        const int toff = (tile_first + 16 * j) & (block_size - 1);
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(cache) + (int64_t)blk * block_stride, 0, 0x7FFFFFFF, 0x00020000);
        // The scheduling barriers keep the ring's loads in program order, which is what
        // lets each wait below count only the loads of later tiles.
        __builtin_amdgcn_sched_barrier(0);
        issue_tile<LAYOUT>(r, rsrc, toff * num_kv_heads * (LAYOUT == 0 ? kSoaRecord : kAosSlot),
                           toff * 2, off);
        __builtin_amdgcn_sched_barrier(0);
    };
    // Stage j: softmax of tile j (scores computed by the previous stage), then one
    // branch-free block with PV of tile j and QK^T of tile j+1, so the two MFMA streams
    // and the decode VALU work interleave.  QK^T of the stage after the chunk's last
    // tile reads a clamped (valid) tile and its scores are discarded.
    TileScores<NSET> sc;
    auto stage = [&](const RawTile<LAYOUT> &cur, const RawTile<LAYOUT> &nxt, int j) {
        const TileRegs t = decode_tile<LAYOUT>(cur, off);
        const int t0 = tile_first + 16 * j;
        const int tok0 = t0 + 4 * u;
        float pw[NSET][4];
        if (t0 >= rng.start && t0 + 16 <= rng.end)
            softmax_tile<LAYOUT, NSET, false>(sc, t, st, pw, tok0, rng.start, rng.end);
        else
            softmax_tile<LAYOUT, NSET, true>(sc, t, st, pw, tok0, rng.start, rng.end);
        pv_tile<NSET>(t, pw, st);
        qk_tile<LAYOUT, NSET>(decode_tile<LAYOUT>(nxt, off).k, ktab, q, sc);
    };

    // Tiles in chunks of 64 (one block-table entry per lane); within a chunk a 4-slot
    // register ring keeps the loads of the next tiles in flight: each slot is refilled
    // right after its tile is consumed.  Every ring load and every stage is
    // unconditional -- past the chunk's last tile a load re-reads that tile (an L2 hit)
    // and the stage masks all of its tokens -- so all paths issue the same loads in the
    // same order and each wait counts exactly the loads of later tiles.
    for (int j0 = 0; j0 < ntiles; j0 += 64) {
        const int n = min(64, ntiles - j0);
        const int last = j0 + n - 1;
        const int bt_val = bt[(tile_first + 16 * (j0 + min(lane, n - 1))) >> block_size_log2];
        RawTile<LAYOUT> r0, r1, r2, r3;
        issue(r0, bt_val, j0);
        issue(r1, bt_val, min(j0 + 1, last));
        issue(r2, bt_val, min(j0 + 2, last));
        issue(r3, bt_val, min(j0 + 3, last));
        qk_tile<LAYOUT, NSET>(decode_tile<LAYOUT>(r0, off).k, ktab, q, sc);
        int j = j0;
        do {
            stage(r0, r1, j);
            issue(r0, bt_val, min(j + 4, last));
            stage(r1, r2, j + 1);
            issue(r1, bt_val, min(j + 5, last));
            stage(r2, r3, j + 2);
            issue(r2, bt_val, min(j + 6, last));
            stage(r3, r0, j + 3);
            issue(r3, bt_val, min(j + 7, last));
            j += 4;
        } while (j <= last);
    }

    // ---- merge the four slots u and write this split's rows
#pragma unroll
    for (int set = 0; set < NSET; ++set) {
        float mx = fmaxf(st.m[set], __shfl_xor(st.m[set], 16, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        const float f = st.m[set] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(st.m[set] - mx);
        float lt = f * st.l[set];
        lt += __shfl_xor(lt, 16, kWave);
        lt += __shfl_xor(lt, 32, kWave);
        const float zf = f * st.z[set];
        const float safe_l = lt > 0.f ? lt : 1.f;
        const float inv = 1.f / safe_l;
        float *row = mid_o + (((int64_t)b * num_q_heads + kvh * G + 4 * set + c) * num_splits + sid) *
                                 (kHeadDim + 1);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float o = f * st.acc[set][k][r] + zf;
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
