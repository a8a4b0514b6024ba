// Stage1, matrix-core kernel (gfx950): one wave64 per (split, kv-head, sequence),
// GQA group G = 4 * NSET, 16-token tiles aligned to the KV block.
//
// Lane l = 16u + 4v + c (u, v, c in 0..3).  MFMA block = l / 4 = 4u + v, in-block
// index = c.  All products run on v_mfma_f32_4x4x1f32 (fp32 operands, 16 blocks); its
// 4x4 shape puts 4 tokens or 4 dims against the 4 heads of a head set, so the GQA
// group costs no padding.  On gfx950 vector instructions do not overlap fp32 MFMAs,
// so the layout is chosen to keep the vector work per tile small.
//
// QK^T of a tile (tokens 4u .. 4u+3 in lane group u):
//   lane (u,v,c) loads the 16 K code bytes of token 4u + ((c + v) & 3), dims 32v ..
//   32v+31.  A[block (u,v)][row i] = K[4u + ((i + v) & 3)][32v + s] (lane (u,v,i)),
//   B[block][col j] = q[head j][32v + s], broadcast from lane group s % 4 by the
//   B lane-group pattern (blgp = 4 + s % 4): lane (g,v,c) holds q[c][32v + 4k + g] in
//   register k.  32 MFMAs (one per dim of the group) leave in lane (u,v,c) register i
//   the dot over dim group v of token 4u + ((i + v) & 3) with head c.  The centroids
//   come from a 256-entry LDS table indexed by the packed code byte (entry = (c[low
//   nibble], c[high nibble])): one ds_read_b64 gives the A operands of two MFMAs.
//   Because of the rotation, register k of lane (u, v-k, c) holds token 4u+v's dot
//   over group v-k, so three DPP row rotations (by 4, 8, 12 lanes) sum the full score
//   of token 4u + v, head c into lane (u,v,c): one score per lane, no duplicates.
// Softmax: lane (u,v,c) owns token 4u+v, head c.  Slot (u, c) (four lanes v) keeps a
//   running max m; the max only moves when a score exceeds it by more than
//   kRescaleLog2 (p <= 2^8), so the rescale branch is rare after a slot's first tile.
//   Each lane accumulates its own l and z (z = sum p * V zero); slots merge at the end.
// PV of the tile, step i (token 4u + i), 8 MFMAs k = 0..7:
//   A[block (u,v)][row h] = p[head h][4u + i] * V scale   -- the A operand of block
//     (u, i), broadcast to the four blocks of lane group u (cbsz = 2, abid = i), i.e.
//     exactly where the softmax left it;
//   B[block (u,v)][col j] = code[4u + i][32v + 8j + k]    -- lane (u,v,j) loads the V
//     dword of token 4u+i at dims 32v + 8j .. +7;
//   result lane (u,v,j) reg h += O[head h][32v + 8j + k] (32 accumulators per set).
//   V codes are converted two at a time with v_cvt_pk_f32_fp8: a byte n < 16 read as
//   fp8 (e4m3) is exactly n * 2^-9; the power-of-two factor is undone at the end.
//
// Schedule: stage j = softmax of tile j, then PV of tile j together with QK^T of tile
// j+1 in one branch-free block (software pipelining across tiles).
//
// Memory: the block-table entries of up to 64 tiles are read once (one lane per tile)
// and broadcast with readlane.  A 4-slot register ring keeps the loads of the next
// tiles in flight.  Loads are buffer loads off a per-tile descriptor whose base is the
// KV block (offsets are per-lane constants), plain and unconditional, so the
// compiler's wait before each tile is exact.
#pragma once
#include "tq4_device.h"

namespace tq4 {

constexpr float kRescaleLog2 = 8.0f;

template <int CTRL> __device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}
// DPP row_ror:N -- lane r of a 16-lane row reads lane (r - N) mod 16.
constexpr int kRor4 = 0x124, kRor8 = 0x128, kRor12 = 0x12C;
// Sum / max over the four lanes of a 16-lane row that share (lane & 3).
__device__ __forceinline__ float row_group_sum(float x) {
    x += dpp<kRor8>(x);
    x += dpp<kRor4>(x);
    return x;
}
__device__ __forceinline__ float row_group_max(float x) {
    x = fmaxf(x, dpp<kRor8>(x));
    return fmaxf(x, dpp<kRor4>(x));
}
// Value of quad lane Q broadcast to the whole quad.
template <int Q> __device__ __forceinline__ float quad_bcast(float x) {
    return dpp<(Q | (Q << 2) | (Q << 4) | (Q << 6))>(x);
}

// B taken from lane group G (lanes 16G .. 16G+15) for all four groups.
template <int G> __device__ __forceinline__ floatx4 mfma_f32_bcast(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 4 + G);
}
// A taken from block I of each lane group (cbsz = 2, abid = I).
template <int I> __device__ __forceinline__ floatx4 mfma_f32_abcast(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 2, I, 0);
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

// Per-lane byte offsets inside one KV block (fixed for a kernel instance).
struct LaneOffsets {
    uint32_t k;     // K bytes of token 4u + ((c+v) & 3), dims 32v ..
    uint32_t v[4];  // V dword of token 4u + i, dims 32v + 8c ..
    uint32_t m;     // SoA: norm of token 4u + v; AoS: slot of token 4u + v
    uint32_t mf;    // SoA: distance between the three metadata arrays
};

template <int LAYOUT>
__device__ __forceinline__ LaneOffsets lane_offsets(int u, int v, int c, int kvh, int hk,
                                                    int block_size) {
    LaneOffsets o;
    const int kt = 4 * u + ((c + v) & 3);
    const int st = 4 * u + v;
    if (LAYOUT == 0) {
        o.k = (kt * hk + kvh) * kSoaRecord + 16 * v;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            o.v[i] = ((4 * u + i) * hk + kvh) * kSoaRecord + kHalfD + 16 * v + 4 * c;
        o.m = block_size * hk * kSoaRecord + (kvh * 3 * block_size + st) * 2;
        o.mf = block_size * 2;
    } else {
        o.k = (kt * hk + kvh) * kAosSlot + 16 * v;  // 2-byte aligned
#pragma unroll
        for (int i = 0; i < 4; ++i)
            o.v[i] = ((4 * u + i) * hk + kvh) * kAosSlot + kHalfD + 2 + 16 * v + 4 * c;
        o.m = (st * hk + kvh) * kAosSlot;
        o.mf = 0;
    }
    return o;
}

// Raw loads of one tile (plain loads, so the compiler tracks their completion).
template <int LAYOUT> struct RawTile;
template <> struct RawTile<0> {
    uint4 k;
    uint32_t v[4];
    uint32_t norm, scale, zero;  // fp16 bits of token 4u + v
};
template <> struct RawTile<1> {
    uint32_t k[5];  // aligned dwords around the (2-byte aligned) K bytes
    uint2 v[4];     // aligned dword pairs around each V dword
    uint32_t norm, scale, zero;
};

// Decoded view of a tile.
struct TileRegs {
    uint4 k;
    uint32_t v[4];
    uint32_t norm, scale, zero;
};

// Loads of one tile.  rsrc: buffer descriptor based at the KV block; doff / moff: byte
// offsets of the tile's 16-token piece inside the block (data records / SoA metadata).
template <int LAYOUT>
__device__ __forceinline__ void issue_tile(RawTile<LAYOUT> &t, __amdgpu_buffer_rsrc_t rsrc,
                                           int doff, int moff, const LaneOffsets &o) {
    if constexpr (LAYOUT == 0) {
        t.k = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, o.k, doff, 0));
#pragma unroll
        for (int i = 0; i < 4; ++i)
            t.v[i] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, o.v[i], doff, 0);
        t.norm = __builtin_amdgcn_raw_buffer_load_b16(rsrc, o.m, moff, 0);
        t.scale = __builtin_amdgcn_raw_buffer_load_b16(rsrc, o.m + o.mf, moff, 0);
        t.zero = __builtin_amdgcn_raw_buffer_load_b16(rsrc, o.m + 2 * o.mf, moff, 0);
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

template <int LAYOUT>
__device__ __forceinline__ TileRegs decode_tile(const RawTile<LAYOUT> &t, const LaneOffsets &o) {
    TileRegs r;
    if constexpr (LAYOUT == 0) {
        r.k = t.k;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            r.v[i] = t.v[i];
    } else {
        const uint32_t sh = o.k & 3u;
        r.k.x = __builtin_amdgcn_alignbyte(t.k[1], t.k[0], sh);
        r.k.y = __builtin_amdgcn_alignbyte(t.k[2], t.k[1], sh);
        r.k.z = __builtin_amdgcn_alignbyte(t.k[3], t.k[2], sh);
        r.k.w = __builtin_amdgcn_alignbyte(t.k[4], t.k[3], sh);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            r.v[i] = __builtin_amdgcn_alignbyte(t.v[i].y, t.v[i].x, o.v[i] & 3u);
    }
    r.norm = t.norm;
    r.scale = t.scale;
    r.zero = t.zero;
    return r;
}

__device__ __forceinline__ float half_lo(uint32_t w) { return half_bits_to_float(w); }

// Running softmax state of lane (u,v,c): slot (u, head c) shares m across v; l and z are
// the lane's own partial sums; acc[set][k] reg h = O[head h][32v + 8c + k] of slot u.
template <int NSET> struct SoftmaxState {
    float negm[NSET];  // -m (exp2 domain); starts at +FLT_MAX: "no token seen yet"
    float l[NSET], z[NSET];
    floatx4 acc[NSET][8];
};

// q in the exp2 domain: lane (g,v,c) holds q[head 4*set + c][32v + 4k + g] in v[set][k].
template <int NSET> struct QOperands {
    float v[NSET][8];
};

// Dots of one tile (one MFMA chain per head set) and, for AoS, the lane's share of
// ||c[idx]||^2 of its K token.
template <int NSET> struct TileScores {
    floatx4 sc[NSET];
    float csq_part;
};

template <int LAYOUT, int NSET>
__device__ __forceinline__ void qk_tile(const uint4 &k, const typename KEntry<LAYOUT>::type *ktab,
                                        const QOperands<NSET> &q, TileScores<NSET> &s) {
#pragma unroll
    for (int set = 0; set < NSET; ++set)
        s.sc[set] = floatx4{0.f, 0.f, 0.f, 0.f};
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
                s.sc[set] = mfma_f32_bcast<2>(e.x, q.v[set][bidx >> 1], s.sc[set]);
                s.sc[set] = mfma_f32_bcast<3>(e.y, q.v[set][bidx >> 1], s.sc[set]);
            } else {
                s.sc[set] = mfma_f32_bcast<0>(e.x, q.v[set][bidx >> 1], s.sc[set]);
                s.sc[set] = mfma_f32_bcast<1>(e.y, q.v[set][bidx >> 1], s.sc[set]);
            }
        }
    }
}

// Full score of token 4u+v (head c) from the rotated partial dots.
__device__ __forceinline__ float gather_score(const floatx4 &sc) {
    float s = sc[0] + dpp<kRor4>(sc[1]);
    s += dpp<kRor8>(sc[2]);
    return s + dpp<kRor12>(sc[3]);
}

// ||c[idx]||^2 of token 4u+v from the per-lane shares (lane (v', c') holds the share of
// token 4u + ((c' + v') & 3) over dim group v').
__device__ __forceinline__ float gather_csq(float x) {
    float s = quad_bcast<0>(x);
    s += dpp<kRor4>(quad_bcast<1>(x));
    s += dpp<kRor8>(quad_bcast<2>(x));
    return s + dpp<kRor12>(quad_bcast<3>(x));
}

// Softmax of one tile -> PV weights pw (p * V scale).  `valid` is false for tokens outside
// the split (only boundary tiles have any).
template <int LAYOUT, int NSET>
__device__ __forceinline__ void softmax_tile(const TileScores<NSET> &s, const TileRegs &t,
                                             SoftmaxState<NSET> &st, float (&pw)[NSET],
                                             bool boundary, bool valid) {
    const _Float16 scale_h = __builtin_bit_cast(_Float16, (unsigned short)t.scale);
    const _Float16 zero_h = __builtin_bit_cast(_Float16, (unsigned short)t.zero);
    float norm;
    if constexpr (LAYOUT == 0) {
        norm = (float)__builtin_bit_cast(_Float16, (unsigned short)t.norm);
    } else {
        const float csq = gather_csq(s.csq_part);
        norm = half_lo(t.norm) * __builtin_amdgcn_rsqf(csq + 1e-16f);
    }
#pragma unroll
    for (int set = 0; set < NSET; ++set) {
        const float dot = gather_score(s.sc[set]);
        float s2 = fmaf(dot, norm, st.negm[set]);  // score - m
        if (boundary)
            s2 = valid ? s2 : -INFINITY;
        const float tmax = row_group_max(s2);
        const bool need = tmax > kRescaleLog2;
        if (__builtin_expect(__any(need), 0)) {
            // New slot max from the exact scores (s2 is inexact while -m = FLT_MAX).
            float sn = dot * norm;
            if (boundary)
                sn = valid ? sn : -INFINITY;
            const float mt = row_group_max(sn);
            const float negm_new = need ? -mt : st.negm[set];
            // exp2(m_old - m_new): 1 for slots that keep their max, 0 for a first token
            const float alpha = __builtin_amdgcn_exp2f(negm_new - st.negm[set]);
            const float a0 = quad_bcast<0>(alpha), a1 = quad_bcast<1>(alpha);
            const float a2 = quad_bcast<2>(alpha), a3 = quad_bcast<3>(alpha);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                st.acc[set][k][0] *= a0;
                st.acc[set][k][1] *= a1;
                st.acc[set][k][2] *= a2;
                st.acc[set][k][3] *= a3;
            }
            st.l[set] *= alpha;
            st.z[set] *= alpha;
            st.negm[set] = negm_new;
            s2 = sn + negm_new;
        }
        const float p = __builtin_amdgcn_exp2f(s2);
        st.l[set] += p;
        st.z[set] = fmaf(p, (float)zero_h, st.z[set]);
        pw[set] = p * (float)scale_h;
    }
}

// PV of one tile on the matrix cores: token 4u+i's weights come from block (u, i).
template <int NSET>
__device__ __forceinline__ void pv_tile(const TileRegs &t, const float (&pw)[NSET],
                                        SoftmaxState<NSET> &st) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = t.v[i] & 0x0F0F0F0Fu;         // codes of dims 8c + 0, 2, 4, 6
        const uint32_t hi = (t.v[i] >> 4) & 0x0F0F0F0Fu;  // codes of dims 8c + 1, 3, 5, 7
        const auto c02 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);
        const auto c46 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
        const auto c13 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
        const auto c57 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
        const float code[8] = {c02[0], c13[0], c02[1], c13[1], c46[0], c57[0], c46[1], c57[1]};
#pragma unroll
        for (int set = 0; set < NSET; ++set) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                switch (i) {
                case 0: st.acc[set][k] = mfma_f32_abcast<0>(pw[set], code[k], st.acc[set][k]); break;
                case 1: st.acc[set][k] = mfma_f32_abcast<1>(pw[set], code[k], st.acc[set][k]); break;
                case 2: st.acc[set][k] = mfma_f32_abcast<2>(pw[set], code[k], st.acc[set][k]); break;
                default: st.acc[set][k] = mfma_f32_abcast<3>(pw[set], code[k], st.acc[set][k]); break;
                }
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
        st.negm[set] = __FLT_MAX__;
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
    // lane's softmax token relative to the split start, at tile 0
    const int rel0 = tile_first + 4 * u + v - rng.start;
    const uint32_t span = (uint32_t)(rng.end - rng.start);
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
    // branch-free block with PV of tile j and QK^T of tile j+1, so the MFMA streams and
    // the decode work interleave.  QK^T after the chunk's last tile reads a clamped
    // (valid) tile and its scores are discarded.
    TileScores<NSET> sc;
    auto stage = [&](const RawTile<LAYOUT> &cur, const RawTile<LAYOUT> &nxt, int j) {
        const TileRegs t = decode_tile<LAYOUT>(cur, off);
        const int t0 = tile_first + 16 * j;
        const bool boundary = !(t0 >= rng.start && t0 + 16 <= rng.end);
        const bool valid = (uint32_t)(rel0 + 16 * j) < span;
        float pw[NSET];
        softmax_tile<LAYOUT, NSET>(sc, t, st, pw, boundary, valid);
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
    // fp8 decode factor: a V code n was accumulated as n * code_unit
    const float inv_code_unit = 1.0f / __builtin_amdgcn_cvt_pk_f32_fp8(1, false)[0];
#pragma unroll
    for (int set = 0; set < NSET; ++set) {
        // slot (u, head c): max, and l / z summed over the slot's four lanes v
        const float m = -st.negm[set];
        float mx = fmaxf(m, __shfl_xor(m, 16, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        const float f = __builtin_amdgcn_exp2f(m - mx);  // 0 for a slot with no token
        float lt = f * row_group_sum(st.l[set]);
        lt += __shfl_xor(lt, 16, kWave);
        lt += __shfl_xor(lt, 32, kWave);
        float zt = f * row_group_sum(st.z[set]);
        zt += __shfl_xor(zt, 16, kWave);
        zt += __shfl_xor(zt, 32, kWave);
        const float safe_l = lt > 0.f ? lt : 1.f;
        const float inv = 1.f / safe_l;
        // per-head factors for the accumulator registers (reg h = head h)
        const float fh[4] = {quad_bcast<0>(f), quad_bcast<1>(f), quad_bcast<2>(f),
                             quad_bcast<3>(f)};
        const float zh[4] = {quad_bcast<0>(zt), quad_bcast<1>(zt), quad_bcast<2>(zt),
                             quad_bcast<3>(zt)};
        const float ih[4] = {quad_bcast<0>(inv), quad_bcast<1>(inv), quad_bcast<2>(inv),
                             quad_bcast<3>(inv)};
        // lane (u,v,c) writes head 4*set + u, dims 32v + 8c .. +7
        float *row = mid_o +
                     (((int64_t)b * num_q_heads + kvh * G + 4 * set + u) * num_splits + sid) *
                         (kHeadDim + 1);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            float out = 0.f;
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                float o = fh[h] * inv_code_unit * st.acc[set][k][h];
                o += __shfl_xor(o, 16, kWave);
                o += __shfl_xor(o, 32, kWave);
                if (h == u)
                    out = (o + zh[h]) * ih[h];
            }
            row[32 * v + 8 * c + k] = out;
        }
        if (lane < 4) {
            float *lrow = mid_o + (((int64_t)b * num_q_heads + kvh * G + 4 * set + c) * num_splits +
                                   sid) * (kHeadDim + 1);
            lrow[kHeadDim] = mx * kLn2 + logf(safe_l);
        }
    }
}

}  // namespace tq4
