// Stage1, matrix-core kernel (gfx950): one wave64 per run of splits of one (kv-head,
// sequence), GQA group G = 4 * NSET, 16-token tiles aligned to the KV block.
//
// Lane l = 16u + 4v + c (u, v, c in 0..3).  MFMA block = l / 4 = 4u + v, in-block
// index = c.  Products run on v_mfma_f32_4x4x4f16 (16 blocks of 4x4, K = 4, fp32
// accumulate); the 4x4 shape puts 4 tokens or 4 dims against the 4 heads of a head set,
// so the GQA group costs no padding.  fp32 accuracy comes from splitting each fp32
// factor into f16 hi + lo parts (x = hi + lo to ~2^-22): every product of interest is
// formed from its parts in the MFMA's K dimension.  (On gfx950 vector instructions do
// not issue while an fp32 MFMA runs; f16 MFMAs leave room for them.)
//
// QK^T of a tile (tokens 4u .. 4u+3 in lane group u):
//   lane (u,v,c) loads the 16 K code bytes of token 4u + ((c + v) & 3), dims 32v ..
//   32v+31.  Per code byte b (dims d = 32v+2b, d' = d+1) two MFMAs:
//     A[block (u,v)][row i][k] = (c_hi[d], c_hi[d'], c_lo[d], c_lo[d'])  of token
//       4u + ((i + v) & 3) (lane (u,v,i)) -- one ds_read_b64 of a 256-entry LDS table
//       indexed by the packed byte;
//     B[k][col j] = (q_hi[d], q_hi[d'], q_hi[d], q_hi[d']) resp. the q_lo parts of head
//       j, broadcast from lane group b % 4 by the B lane-group pattern (blgp = 4 + b%4):
//       lane (g,v,c) holds q[c][32v + 8k + 2g, +1] for k = 0..3;
//   so sum_k A B = c[d] q[d] + c[d'] q[d'] (hi and lo chains accumulate separately).
//   After 32 MFMAs lane (u,v,c) register i holds the dot over dim group v of token
//   4u + ((i + v) & 3) with head c.  Because of the rotation, register k of lane
//   (u, v-k, c) holds token 4u+v's dot over group v-k, so three DPP row rotations (by 4,
//   8, 12 lanes) sum the full score of token 4u + v, head c into lane (u,v,c): one score
//   per lane, no duplicates.
// Softmax: lane (u,v,c) owns token 4u+v, head c.  Slot (u, c) (four lanes v) keeps a
//   running max m; the max only moves when a score exceeds it by more than
//   kRescaleLog2 (p <= 2^8), so the rescale branch is rare after a slot's first tile.
//   Each lane accumulates its own l and z (z = sum p * V zero); slots merge at the end.
// PV of the tile, per dim k of the lane (dims 32v + 8c + k), two MFMAs (hi, lo):
//   A[block (u,v)][row h][t] = w_hi[head h][token 4u+t] (resp. w_lo), w = p * V scale --
//     the A operand of block (u, 3), broadcast to the four blocks of lane group u
//     (cbsz = 2, abid = 3); lane (u,3,h) gathers the four tokens' w with DPP rotations;
//   B[t][col j] = code[4u + t][32v + 8j + k] as an f16 bit pattern (the denormal
//     code * 2^-24; one v_perm_b32 packs two tokens' codes), lane (u,v,j) having loaded
//     the V dword of each token 4u+t at dims 32v + 8j .. +7;
//   result lane (u,v,j) reg h += O[head h][32v + 8j + k] * 2^-24 (32 accumulators / set).
//   w < 65504 is required: p <= 2^8 and V scale < 255.
//
// Schedule: stage j = softmax of tile j, then PV of tile j together with QK^T of tile
// j+1 in one branch-free block (software pipelining across tiles).
//
// Memory: the block-table entries of up to 64 tiles are read once (one lane per tile)
// and broadcast with readlane.  A register ring keeps the loads of the next tiles in
// flight.  Loads are buffer loads off a per-tile descriptor whose base is the KV block
// (offsets are per-lane constants), plain and unconditional, so the compiler's wait
// before each tile is exact.
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

typedef _Float16 halfx4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ halfx4 as_halfx4(uint32_t lo, uint32_t hi) {
    return __builtin_bit_cast(halfx4, uint2{lo, hi});
}
// B taken from lane group G (lanes 16G .. 16G+15) for all four groups.
template <int G> __device__ __forceinline__ floatx4 mfma_f16_bcast(halfx4 a, halfx4 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 0, 0, 4 + G);
}
// A taken from block I of each lane group (cbsz = 2, abid = I).
template <int I> __device__ __forceinline__ floatx4 mfma_f16_abcast(halfx4 a, halfx4 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 2, I, 0);
}
// f16 hi + lo parts of an fp32 value, packed (hi in bits 0..15, lo in 16..31); both
// parts are rounded toward zero, hi + lo = x to ~2^-20 relative.
__device__ __forceinline__ uint32_t split_f16(float x) {
    const auto h = __builtin_amdgcn_cvt_pkrtz(x, 0.f);
    const float r = x - (float)h[0];
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x, r));
}

// K-code table entry for one packed byte (low nibble = even dim d, high nibble = odd
// dim d'): the f16 parts (c_hi[lo], c_hi[hi], c_lo[lo], c_lo[hi]) -- the A operand of
// both QK^T MFMAs of the byte; AoS adds c[lo]^2 + c[hi]^2 (fp32) for the norm
// correction.
template <int LAYOUT> struct KEntry;
template <> struct KEntry<0> { typedef uint2 type; };
template <> struct KEntry<1> { typedef uint4 type; };

template <int LAYOUT>
__device__ __forceinline__ void build_key_table(typename KEntry<LAYOUT>::type *tbl,
                                                const float *pair_lut, int lane) {
    for (int e = lane; e < 256; e += kWave) {
        const int lo = e & 15, hi = e >> 4;
        const float c_lo = pair_lut[2 * (lo * 16 + hi)];      // row (lo, hi) = (c[lo], c[hi])
        const float c_hi = pair_lut[2 * (lo * 16 + hi) + 1];
        const uint32_t p_lo = split_f16(c_lo), p_hi = split_f16(c_hi);
        const uint32_t his = (p_lo & 0xFFFFu) | (p_hi << 16);   // (c_hi[lo], c_hi[hi])
        const uint32_t los = (p_lo >> 16) | (p_hi & 0xFFFF0000u);  // (c_lo[lo], c_lo[hi])
        if constexpr (LAYOUT == 0)
            tbl[e] = uint2{his, los};
        else
            tbl[e] = uint4{his, los, __builtin_bit_cast(uint32_t, c_lo * c_lo + c_hi * c_hi), 0u};
    }
}

// Per-lane byte offsets inside one KV block (fixed for a kernel instance).  The
// per-token steps that are the same for every lane (V dword of token 4u+i relative
// to token 4u, the three SoA metadata arrays) travel in the loads' scalar offsets.
struct LaneOffsets {
    uint32_t k;   // K bytes of token 4u + ((c+v) & 3), dims 32v ..
    uint32_t v0;  // V dword of token 4u, dims 32v + 8c ..; token 4u+i adds i * tok_stride
    uint32_t m;   // SoA: norm of token 4u + v; AoS: slot of token 4u + v
    int tok_stride;  // bytes between consecutive tokens of one kv-head
    int mf;          // SoA: bytes between the three metadata arrays
    int v_shift;     // AoS: v0 & 3 (the same in every lane)
};

template <int LAYOUT>
__device__ __forceinline__ LaneOffsets lane_offsets(int u, int v, int c, int kvh, int hk,
                                                    int block_size) {
    LaneOffsets o;
    const int kt = 4 * u + ((c + v) & 3);
    const int st = 4 * u + v;
    const int rec = LAYOUT == 0 ? kSoaRecord : kAosSlot;
    o.tok_stride = hk * rec;
    o.k = (kt * hk + kvh) * rec + 16 * v;  // AoS: 2-byte aligned
    o.v0 = (4 * u * hk + kvh) * rec + kHalfD + (LAYOUT == 0 ? 0 : 2) + 16 * v + 4 * c;
    if (LAYOUT == 0) {
        o.m = block_size * hk * kSoaRecord + (kvh * 3 * block_size + st) * 2;
        o.mf = block_size * 2;
        o.v_shift = 0;
    } else {
        o.m = (st * hk + kvh) * kAosSlot;
        o.mf = 0;
        o.v_shift = (kvh * kAosSlot + kHalfD + 2) & 3;  // lane terms are multiples of 4
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
            t.v[i] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, o.v0, doff + i * o.tok_stride, 0);
        t.norm = __builtin_amdgcn_raw_buffer_load_b16(rsrc, o.m, moff, 0);
        t.scale = __builtin_amdgcn_raw_buffer_load_b16(rsrc, o.m, moff + o.mf, 0);
        t.zero = __builtin_amdgcn_raw_buffer_load_b16(rsrc, o.m, moff + 2 * o.mf, 0);
    } else {
        const uint32_t ka = o.k & ~3u;
        const auto k03 = __builtin_amdgcn_raw_buffer_load_b128(rsrc, ka, doff, 0);
        t.k[0] = k03[0];
        t.k[1] = k03[1];
        t.k[2] = k03[2];
        t.k[3] = k03[3];
        t.k[4] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, ka + 16, doff, 0);
        // token 4u+i's V dword starts sh = (v_shift + i * tok_stride) & 3 bytes past a
        // dword; both offsets below are multiples of 4 and non-negative.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int sh = (o.v_shift + i * o.tok_stride) & 3;
            t.v[i] = __builtin_bit_cast(
                uint2, __builtin_amdgcn_raw_buffer_load_b64(
                           rsrc, o.v0 - o.v_shift, doff + i * o.tok_stride + o.v_shift - sh, 0));
        }
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
            r.v[i] = __builtin_amdgcn_alignbyte(t.v[i].y, t.v[i].x,
                                                (o.v_shift + i * o.tok_stride) & 3);
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

// q in the exp2 domain as B operands: lane (g,v,c), head 4*set + c, dims
// d = 32v + 8k + 2g and d+1: hi[set][k] = (q_hi[d], q_hi[d+1], q_hi[d], q_hi[d+1]),
// lo[set][k] the same with the lo parts.
template <int NSET> struct QOperands {
    halfx4 hi[NSET][4], lo[NSET][4];
};

// Dots of one tile (one MFMA chain per head set) and, for AoS, the lane's share of
// ||c[idx]||^2 of its K token.
template <int NSET> struct TileScores {
    floatx4 sc[NSET], sd[NSET];  // two independent chains: low / high nibbles
    float csq_part;
};

// One K code byte b (dims 2b, 2b+1 of the lane's dim group) into the two QK^T chains.
template <int LAYOUT, int NSET>
__device__ __forceinline__ void qk_byte(int bidx, uint32_t byte, const typename KEntry<LAYOUT>::type *ktab,
                                        const QOperands<NSET> &q, TileScores<NSET> &s) {
    const auto e = ktab[byte];
    const halfx4 a = as_halfx4(e.x, e.y);
    if constexpr (LAYOUT == 1)
        s.csq_part += __builtin_bit_cast(float, e.z);
#pragma unroll
    for (int set = 0; set < NSET; ++set) {
        // dims 2b, 2b+1 = 8k + 2g (+1) with k = b / 4, g = b % 4
        switch (bidx & 3) {
        case 0:
            s.sc[set] = mfma_f16_bcast<0>(a, q.hi[set][bidx >> 2], s.sc[set]);
            s.sd[set] = mfma_f16_bcast<0>(a, q.lo[set][bidx >> 2], s.sd[set]);
            break;
        case 1:
            s.sc[set] = mfma_f16_bcast<1>(a, q.hi[set][bidx >> 2], s.sc[set]);
            s.sd[set] = mfma_f16_bcast<1>(a, q.lo[set][bidx >> 2], s.sd[set]);
            break;
        case 2:
            s.sc[set] = mfma_f16_bcast<2>(a, q.hi[set][bidx >> 2], s.sc[set]);
            s.sd[set] = mfma_f16_bcast<2>(a, q.lo[set][bidx >> 2], s.sd[set]);
            break;
        default:
            s.sc[set] = mfma_f16_bcast<3>(a, q.hi[set][bidx >> 2], s.sc[set]);
            s.sd[set] = mfma_f16_bcast<3>(a, q.lo[set][bidx >> 2], s.sd[set]);
            break;
        }
    }
}

template <int NSET> __device__ __forceinline__ void clear_scores(TileScores<NSET> &s) {
#pragma unroll
    for (int set = 0; set < NSET; ++set) {
        s.sc[set] = floatx4{0.f, 0.f, 0.f, 0.f};
        s.sd[set] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    s.csq_part = 0.f;
}

template <int LAYOUT, int NSET>
__device__ __forceinline__ void qk_tile(const uint4 &k, const typename KEntry<LAYOUT>::type *ktab,
                                        const QOperands<NSET> &q, TileScores<NSET> &s) {
    clear_scores(s);
    const uint32_t kwords[4] = {k.x, k.y, k.z, k.w};
#pragma unroll
    for (int bidx = 0; bidx < 16; ++bidx)
        qk_byte<LAYOUT, NSET>(bidx, (kwords[bidx >> 2] >> (8 * (bidx & 3))) & 0xFFu, ktab, q, s);
}

// Full score of token 4u+v (head c) from the rotated partial dots.
__device__ __forceinline__ float gather_score(const floatx4 &sc, const floatx4 &sd) {
    const floatx4 t = sc + sd;
    float s = t[0] + dpp<kRor4>(t[1]);
    s += dpp<kRor8>(t[2]);
    return s + dpp<kRor12>(t[3]);
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
        const float dot = gather_score(s.sc[set], s.sd[set]);
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

template <int CTRL> __device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, CTRL, 0xF, 0xF, true);
}

// PV A operands of one head set: the hi / lo f16 parts of w = p * V scale of tokens
// 4u .. 4u+3 (lane (u,3,h) -- block (u,3) -- is the one the MFMAs read).
__device__ __forceinline__ void pv_weights(float w, halfx4 &a_hi, halfx4 &a_lo) {
    const uint32_t t3 = split_f16(w);           // own token 4u+v (v = 3 in block (u,3))
    const uint32_t t2 = dpp_u32<kRor4>(t3);     // token 4u+v-1
    const uint32_t t1 = dpp_u32<kRor8>(t3);
    const uint32_t t0 = dpp_u32<kRor12>(t3);
    a_hi = as_halfx4(__builtin_amdgcn_perm(t1, t0, 0x05040100u), __builtin_amdgcn_perm(t3, t2, 0x05040100u));
    a_lo = as_halfx4(__builtin_amdgcn_perm(t1, t0, 0x07060302u), __builtin_amdgcn_perm(t3, t2, 0x07060302u));
}

// PV of the current tile interleaved with QK^T of the next tile: per K byte two QK^T
// MFMAs and one PV MFMA (dim k = b / 2; hi part for even b, lo part for odd b), so the
// dependent chains are spaced by independent work.
template <int LAYOUT, int NSET>
__device__ __forceinline__ void pv_qk_tile(const TileRegs &t, const float (&pw)[NSET],
                                           SoftmaxState<NSET> &st, const uint4 &knext,
                                           const typename KEntry<LAYOUT>::type *ktab,
                                           const QOperands<NSET> &q, TileScores<NSET> &s) {
    halfx4 a_hi[NSET], a_lo[NSET];
#pragma unroll
    for (int set = 0; set < NSET; ++set)
        pv_weights(pw[set], a_hi[set], a_lo[set]);
    // codes of the even (low nibble) and odd (high nibble) dims of tokens 4u+i
    uint32_t even[4], odd[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        even[i] = t.v[i] & 0x0F0F0F0Fu;
        odd[i] = (t.v[i] >> 4) & 0x0F0F0F0Fu;
    }
    clear_scores(s);
    const uint32_t kwords[4] = {knext.x, knext.y, knext.z, knext.w};
    halfx4 codes;
#pragma unroll
    for (int bidx = 0; bidx < 16; ++bidx) {
        qk_byte<LAYOUT, NSET>(bidx, (kwords[bidx >> 2] >> (8 * (bidx & 3))) & 0xFFu, ktab, q, s);
        const int k = bidx >> 1;  // dim 32v + 8c + k: byte k / 2 of the dword, nibble k % 2
        if ((bidx & 1) == 0) {
            const uint32_t sel = (uint32_t)(k >> 1) | 0x0C00u | ((uint32_t)(4 + (k >> 1)) << 16) | 0x0C000000u;
            const uint32_t *m = (k & 1) ? odd : even;
            codes = as_halfx4(__builtin_amdgcn_perm(m[1], m[0], sel), __builtin_amdgcn_perm(m[3], m[2], sel));
        }
#pragma unroll
        for (int set = 0; set < NSET; ++set)
            st.acc[set][k] = mfma_f16_abcast<3>((bidx & 1) ? a_lo[set] : a_hi[set], codes, st.acc[set][k]);
    }
}

// Lane-pair exchanges of gfx950 (v_permlane32_swap / v_permlane16_swap).
__device__ __forceinline__ uint32_t fbits(float x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ float bitsf(uint32_t x) { return __builtin_bit_cast(float, x); }
// Sum of x over lanes l and l ^ 32 (resp. l ^ 16), in every lane.
__device__ __forceinline__ float sum_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(fbits(x), fbits(x), false, false);
    return bitsf(r[0]) + bitsf(r[1]);
}
__device__ __forceinline__ float sum_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(fbits(x), fbits(x), false, false);
    return bitsf(r[0]) + bitsf(r[1]);
}
__device__ __forceinline__ float max_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(fbits(x), fbits(x), false, false);
    return fmaxf(bitsf(r[0]), bitsf(r[1]));
}
__device__ __forceinline__ float max_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(fbits(x), fbits(x), false, false);
    return fmaxf(bitsf(r[0]), bitsf(r[1]));
}
// Reduce-scatter over lane halves: lanes 0..31 get a[l] + a[l+32], lanes 32..63 get
// c[l-32] + c[l].
__device__ __forceinline__ float rs_xor32(float a, float c) {
    const auto r = __builtin_amdgcn_permlane32_swap(fbits(a), fbits(c), false, false);
    return bitsf(r[0]) + bitsf(r[1]);
}
// Same over 16-lane rows: even rows get a summed with the next row, odd rows get c
// summed with the previous row.
__device__ __forceinline__ float rs_xor16(float a, float c) {
    const auto r = __builtin_amdgcn_permlane16_swap(fbits(a), fbits(c), false, false);
    return bitsf(r[0]) + bitsf(r[1]);
}

// Merge the four slots u of one split and write its rows: lane (u,v,c) writes head
// 4*set + u, dims 32v + 8c .. +7, and lanes 0..3 write the LSE of heads 4*set + c.
template <int NSET>
__device__ __forceinline__ void write_split(const SoftmaxState<NSET> &st, float *__restrict__ mid_o,
                                            int64_t row0, int num_splits, int sid, int u, int v,
                                            int c, int lane, float inv_code_unit) {
#pragma unroll
    for (int set = 0; set < NSET; ++set) {
        // slot (u, head c): max over the slots, then l / z summed over the slot's lanes v
        // and over the slots with their factors
        const float m = -st.negm[set];
        const float mx = max_xor16(max_xor32(m));
        const float f = __builtin_amdgcn_exp2f(m - mx);  // 0 for a slot with no token
        const float lt = sum_xor16(sum_xor32(f * row_group_sum(st.l[set])));
        const float zt = sum_xor16(sum_xor32(f * row_group_sum(st.z[set])));
        const float safe_l = lt > 0.f ? lt : 1.f;
        // head c totals -> the lanes that write head u
        const int src = (lane & ~3) | u;
        const float z_u = __shfl(zt, src, kWave);
        const float inv_u = 1.f / __shfl(safe_l, src, kWave);
        // accumulator register h = head h: scale by slot u's factor for head h
        const float fh0 = quad_bcast<0>(f) * inv_code_unit, fh1 = quad_bcast<1>(f) * inv_code_unit;
        const float fh2 = quad_bcast<2>(f) * inv_code_unit, fh3 = quad_bcast<3>(f) * inv_code_unit;
        float *row = mid_o + ((row0 + 4 * set + u) * num_splits + sid) * (kHeadDim + 1);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const floatx4 a = st.acc[set][k];
            // sum over slots u: heads 0 / 2 and 1 / 3 split across the lane halves, then
            // across rows, leaving head u in lane group u
            const float x = rs_xor32(a[0] * fh0, a[2] * fh2);
            const float y = rs_xor32(a[1] * fh1, a[3] * fh3);
            const float o = rs_xor16(x, y);
            row[32 * v + 8 * c + k] = (o + z_u) * inv_u;
        }
        if (lane < 4) {
            float *lrow = mid_o + ((row0 + 4 * set + c) * num_splits + sid) * (kHeadDim + 1);
            lrow[kHeadDim] = mx * kLn2 + logf(safe_l);
        }
    }
}

// One wave handles a run of consecutive live splits of one (sequence, kv-head).  Their tiles form one stream: split s contributes n_s tiles padded to a
// multiple of 4 stream positions (padding positions re-read the split's last tile and
// mask every token), so split ends fall on 4-stage group boundaries.  The load ring
// and the QK^T pipeline run across split boundaries; after a split's last group the
// wave writes its rows and restarts the softmax state (the first rescale of the next
// split multiplies the old accumulators by 0).  RING tiles are in flight per wave.
template <int LAYOUT, int NSET, int RING>
__global__ __launch_bounds__(kWave) void stage1_mfma_kernel(
    const float *__restrict__ q_rot, const uint8_t *__restrict__ cache,
    const int32_t *__restrict__ block_table, const int32_t *__restrict__ seq_lens,
    const float *__restrict__ pair_lut, float *__restrict__ mid_o, int num_q_heads,
    int num_kv_heads, int block_size_log2, int max_blocks, int64_t block_stride, int num_splits,
    float score_scale_log2) {
    constexpr int G = 4 * NSET;
    const int block_size = 1 << block_size_log2;
    // grid (Hk, W, B): the kv-heads of one (sequence, split run) are dispatched together,
    // so the waves that read the same KV blocks run at about the same time.
    const int kvh = blockIdx.x;
    const int wid = blockIdx.y, nw = gridDim.y;
    const int b = blockIdx.z;
    const int lane = threadIdx.x;
    const int seq_len = seq_lens[b];
    // split partition: L = ceil(len / S); live splits are those with s * L < len
    const int split_len = (seq_len + num_splits - 1) / num_splits;
    // wave x of the W waves of this (sequence, kv-head) takes splits [x * S / W, (x + 1) * S / W)
    const int s_lo = (int)((int64_t)wid * num_splits / nw);
    const int live = split_len > 0 ? min(num_splits, (seq_len + split_len - 1) / split_len) : 0;
    const int s_hi = min((int)((int64_t)(wid + 1) * num_splits / nw), live);
    if (s_lo >= s_hi)
        return;
    const int c = lane & 3;
    const int v = (lane >> 2) & 3;
    const int u = lane >> 4;

    __shared__ typename KEntry<LAYOUT>::type ktab[256];
    build_key_table<LAYOUT>(ktab, pair_lut, lane);

    // q of heads (kvh*G + 4*set + c), dims 32v + 8k + 2u (+1), scaled to the exp2 domain
    QOperands<NSET> q;
#pragma unroll
    for (int set = 0; set < NSET; ++set) {
        const float *qp =
            q_rot + ((int64_t)b * num_q_heads + kvh * G + 4 * set + c) * kHeadDim + 32 * v + 2 * u;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t p0 = split_f16(qp[8 * k] * score_scale_log2);
            const uint32_t p1 = split_f16(qp[8 * k + 1] * score_scale_log2);
            const uint32_t his = (p0 & 0xFFFFu) | (p1 << 16), los = (p0 >> 16) | (p1 & 0xFFFF0000u);
            q.hi[set][k] = as_halfx4(his, his);
            q.lo[set][k] = as_halfx4(los, los);
        }
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

    // stream positions of a split with n tiles: n rounded up to a whole ring turn
    static_assert(RING == 4 || RING == 8, "ring of 4 or 8 tiles");
    auto ring_padded = [](int n) { return (n + RING - 1) & ~(RING - 1); };
    int total = 0;
    for (int s = s_lo; s < s_hi; ++s) {
        const int st0 = s * split_len, en = min(st0 + split_len, seq_len);
        total += ring_padded(((en - 1) >> 4) - (st0 >> 4) + 1);
    }

    const LaneOffsets off = lane_offsets<LAYOUT>(u, v, c, kvh, num_kv_heads, block_size);
    const int32_t *bt = block_table + (int64_t)b * max_blocks;
    const int ktok = 4 * u + v;  // the lane's softmax token within a tile
    const int64_t row0 = (int64_t)b * num_q_heads + kvh * G;
    const float inv_code_unit = 16777216.0f;  // V codes enter the MFMA as n * 2^-24
    __syncthreads();

    // current split (uniform): [cur_start, cur_end), stream position of its end
    int cur = s_lo;
    int cur_start = cur * split_len;
    int cur_end = min(cur_start + split_len, seq_len);
    int cur_stop = ring_padded(((cur_end - 1) >> 4) - (cur_start >> 4) + 1);

    // Issue the loads of stream position j into ring slot r; its block id and tile index
    // sit in lane (j mod 64) of bt_lane / tile_lane.
    auto issue = [&](RawTile<LAYOUT> &r, int bt_lane, int tile_lane, int j) {
        const int blk = __builtin_amdgcn_readlane(bt_lane, j & 63);
        const int toff = (16 * __builtin_amdgcn_readlane(tile_lane, j & 63)) & (block_size - 1);
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(cache) + (int64_t)blk * block_stride, 0, 0x7FFFFFFF, 0x00020000);
        // The scheduling barriers keep the ring's loads in program order, which is what
        // lets each wait below count only the loads of later tiles.
        __builtin_amdgcn_sched_barrier(0);
        issue_tile<LAYOUT>(r, rsrc, toff * num_kv_heads * (LAYOUT == 0 ? kSoaRecord : kAosSlot),
                           toff * 2, off);
        __builtin_amdgcn_sched_barrier(0);
    };
    // Stage j: softmax of position j (scores computed by the previous stage), then one
    // branch-free block with PV of position j and QK^T of position j+1, so the MFMA
    // streams and the decode work interleave.
    TileScores<NSET> sc;
    auto stage = [&](const RawTile<LAYOUT> &cur_t, const RawTile<LAYOUT> &nxt_t, int mask_lane,
                     int j) {
        const TileRegs t = decode_tile<LAYOUT>(cur_t, off);
        const int t0 = 16 * __builtin_amdgcn_readlane(mask_lane, j & 63);
        const bool boundary = !(t0 >= cur_start && t0 + 16 <= cur_end);
        const bool valid = (uint32_t)(t0 + ktok - cur_start) < (uint32_t)(cur_end - cur_start);
        float pw[NSET];
        softmax_tile<LAYOUT, NSET>(sc, t, st, pw, boundary, valid);
        pv_qk_tile<LAYOUT, NSET>(t, pw, st, decode_tile<LAYOUT>(nxt_t, off).k, ktab, q, sc);
    };

    // Stream positions in chunks of 64 (one block-table entry per lane); within a chunk
    // a 4-slot register ring keeps the loads of the next positions in flight: each slot
    // is refilled right after its tile is consumed.  Every ring load and every stage is
    // unconditional -- past the chunk's end a load re-reads its last tile (an L2 hit) --
    // so all paths issue the same loads in the same order and each wait counts exactly
    // the loads of later positions.
    int pos_base = 0;  // stream position where split `cur` starts
    for (int j0 = 0; j0 < total; j0 += 64) {
        const int n = min(64, total - j0);
        const int last = j0 + n - 1;
        // lane i: the tile at stream position j0 + i (clamped to the chunk)
        int tile_lane = 0, mask_lane = 0;
        {
            const int p = j0 + min(lane, n - 1);
            int base = 0;
            for (int s = s_lo; s < s_hi; ++s) {
                const int st0 = s * split_len, en = min(st0 + split_len, seq_len);
                const int tf = st0 >> 4, nt = ((en - 1) >> 4) - tf + 1;
                if (p >= base) {
                    const int o = p - base;
                    tile_lane = tf + min(o, nt - 1);
                    mask_lane = o < nt ? tile_lane : -(1 << 24);  // padding: no valid token
                }
                base += ring_padded(nt);
            }
        }
        const int bt_lane = bt[(16 * tile_lane) >> block_size_log2];
        RawTile<LAYOUT> ring[RING];
#pragma unroll
        for (int k = 0; k < RING; ++k)
            issue(ring[k], bt_lane, tile_lane, min(j0 + k, last));
        qk_tile<LAYOUT, NSET>(decode_tile<LAYOUT>(ring[0], off).k, ktab, q, sc);
        int j = j0;
        while (true) {
            // ring turns up to the end of the current split or of the chunk
            const int stop = min(pos_base + cur_stop, last + 1);
            do {
#pragma unroll
                for (int k = 0; k < RING; ++k) {
                    stage(ring[k], ring[(k + 1) % RING], mask_lane, j + k);
                    issue(ring[k], bt_lane, tile_lane, min(j + k + RING, last));
                }
                j += RING;
            } while (j < stop);
            if (j == pos_base + cur_stop) {
                write_split<NSET>(st, mid_o, row0, num_splits, cur, u, v, c, lane, inv_code_unit);
#pragma unroll
                for (int set = 0; set < NSET; ++set)
                    st.negm[set] = __FLT_MAX__;
                pos_base = j;
                ++cur;
                cur_start = cur * split_len;
                cur_end = min(cur_start + split_len, seq_len);
                cur_stop = ring_padded(((cur_end - 1) >> 4) - (cur_start >> 4) + 1);
            }
            if (j > last)
                break;
        }
    }
}

}  // namespace tq4
