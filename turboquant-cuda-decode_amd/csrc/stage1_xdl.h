// Stage1 on gfx950's full-rate f16 matrix instruction v_mfma_f32_16x16x32_f16: one
// wave64 per run of splits of one (kv-head, sequence), GQA group G = 4 or 8, 16-token
// tiles aligned to the KV block.
//
// Lane l = 16g + n (g = l / 16 in 0..3, n = l % 16).  For a 16x16x32 MFMA, lane (n, g)
// holds A[row n][k-slots 8g .. 8g+7], B[k-slots 8g .. 8g+7][col n], and D[rows 4g .. 4g+3]
// [col n].  fp32 accuracy comes from splitting each fp32 factor into f16 hi + lo parts
// (x = hi + lo to ~2^-20); the parts are placed so that every cross product that
// matters is formed.
//
// Columns / rows that stand for heads: index n -> head n & (G-1), part n >> 3 (0 = hi,
// 1 = lo).  For G = 4 indices 4..7 and 12..15 repeat 0..3 and 8..11.
//
// QK^T of a tile (16 tokens):  lane (n, g) loads token n's 16 code bytes 16g .. 16g+15
//   (dims 32g ..) in one dwordx4; each byte gives (c_hi[lo], c_hi[hi], c_lo[lo],
//   c_lo[hi]) through one ds_read_b64 of a 256-entry LDS table.  MFMA m = 0..7 takes
//   bytes 2m, 2m+1: A[token n][slots] = (c_hi, c_hi, c_lo, c_lo) of each byte's two dims,
//   B[slots][col] = q_part(col)[head(col)] of the same dims (pre-scaled by attn_scale *
//   log2 e), so D[t][col] = sum over dims of (c_hi + c_lo) q_part.  Adding column n ^ 8
//   (DPP row_ror:8) gives the full dot of token 4g + i, head n & (G-1) in register i of
//   every lane.
// Softmax: lane (n, g) owns TPL = G / 4 tokens: 4g + TPL * (n / G) + j, head n & (G-1).
//   The running max m is shared by all lanes of a head and moves only when a score
//   exceeds it by more than kRescaleLogX (p <= 2^8); that branch is rare after a
//   split's first tile, and only the second tile of a pair rescales the accumulators.
//   Each lane accumulates its own l = sum p and z = sum p * V zero.
// PV of a pair of tiles (32 tokens):  A[row][slot s] = w_part(row)[head(row)] of token
//   4g + (s & 3) of tile s / 4, w = p * V scale (gathered from the owning lanes with DPP
//   row rotations);  B[slot s][col n] = V code of the same token at dim 8n + j for MFMA
//   j = 0..7, as an f16 bit pattern (lane (n, g) loads V dword n of tokens 4g .. 4g+3;
//   v_perm_b32 packs two tokens' bytes).  Accumulator 2m takes the low nibbles (dim
//   8n + 2m), accumulator 2m + 1 the whole bytes (dim 8n + 2m plus 16 x dim 8n + 2m + 1),
//   both shifted to the top of the f16 significand (see pv_qk); D rows 4g + r hold part
//   g >> 1 of the sums.
//
// Schedule: stage t = softmax of tile t, then QK^T of tile t + 1; odd stages also run
// the PV of tiles (t-1, t), interleaved with that QK^T.  K loads run 4 tiles ahead of
// their QK^T, V / metadata loads 3-4 tiles ahead of their softmax.
// Output: a finished split's rows go to an LDS image of the wave's part of mid_o, which
// is written out as one contiguous run per head (see SpanCap).
#pragma once
#include <type_traits>
#include "stage2.h"
#include "tq4_device.h"

namespace tq4 {
namespace xdl {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kRescaleLogX = 8.0f;
constexpr int kRor4 = 0x124, kRor8 = 0x128, kRor12 = 0x12C;  // DPP row_ror:N

// DPP row_ror:N -- lane r of a 16-lane row reads lane (r - N) mod 16.
template <int CTRL> __device__ __forceinline__ uint32_t dpp(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, CTRL, 0xF, 0xF, true);
}
template <int CTRL> __device__ __forceinline__ float dppf(float x) {
    return __builtin_bit_cast(float, dpp<CTRL>(__builtin_bit_cast(uint32_t, x)));
}
// Value of quad lane Q broadcast to the whole quad.
template <int Q> __device__ __forceinline__ float quad_bcast(float x) {
    return dppf<(Q | (Q << 2) | (Q << 4) | (Q << 6))>(x);
}
__device__ __forceinline__ uint32_t fbits(float x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ float bitsf(uint32_t x) { return __builtin_bit_cast(float, x); }
__device__ __forceinline__ float sum_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(fbits(x), fbits(x), false, false);
    return bitsf(r[0]) + bitsf(r[1]);
}
__device__ __forceinline__ float sum_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(fbits(x), fbits(x), false, false);
    return bitsf(r[0]) + bitsf(r[1]);
}
// max of two scores, which are never NaN (finite, or -inf for masked tokens): one v_max_f32,
// without the two quieting v_max that fmaxf adds for operands read across lanes
__device__ __forceinline__ float max_score(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ float max_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(fbits(x), fbits(x), false, false);
    return max_score(bitsf(r[0]), bitsf(r[1]));
}
__device__ __forceinline__ float max_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(fbits(x), fbits(x), false, false);
    return max_score(bitsf(r[0]), bitsf(r[1]));
}
// Reduce-scatter over lane halves: lanes 0..31 get a[l] + a[l+32], lanes 32..63 get
// c[l-32] + c[l].
__device__ __forceinline__ float rs_xor32(float a, float c) {
    const auto r = __builtin_amdgcn_permlane32_swap(fbits(a), fbits(c), false, false);
    return bitsf(r[0]) + bitsf(r[1]);
}

// f16 hi + lo parts of an fp32 value, packed (hi in bits 0..15, lo in 16..31): hi + lo =
// x to 2^-22 relative while lo is a normal f16, else to half the f16 denormal step.  hi is
// rounded toward zero (v_cvt_pkrtz, saturating), so lo has the sign of x: measured on
// gfx950, the matrix core sums the eight products of a lane's k-slots with truncation
// relative to the largest of them, and parts of one sign keep that error smallest (the PV
// sums stay all-positive).  lo is rounded to nearest, so the residual error has no
// preferred sign and does not build up over a split's tokens.  |x| must stay below 65504.
__device__ __forceinline__ uint32_t split_f16(float x) {
    auto h = __builtin_amdgcn_cvt_pkrtz(x, 0.f);
    h[1] = (__fp16)(x - (float)h[0]);
    return __builtin_bit_cast(uint32_t, h);
}
__device__ __forceinline__ half8 as_half8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return __builtin_bit_cast(half8, uint4{a, b, c, d});
}
__device__ __forceinline__ floatx4 mfma(half8 a, half8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float half_at(uint32_t w, int hi) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(hi ? (w >> 16) : (w & 0xFFFFu)));
}

// K-code table indexed by one packed byte (low nibble = even dim, high nibble = odd dim):
// entry e = ((c_hi[lo], c_hi[hi]), (c_lo[lo], c_lo[hi])) as two f16 pairs, read with one
// ds_read_b64 straight into half of a QK^T operand; the AoS norm correction sums
// c[lo]^2 + c[hi]^2 from the same entries (f16 dot products into fp32, lookup_tile).
template <int LAYOUT> struct KTable {
    static constexpr int words = 512;
};

// Pair-LUT rows of the lane's table entries e = lane + 64 i (loaded before the build so
// their latency overlaps the first KV loads).
struct LutRows {
    float2 r[256 / kWave];
};
__device__ __forceinline__ LutRows load_lut_rows(const float *pair_lut, int lane) {
    LutRows v;
#pragma unroll
    for (int i = 0; i < 256 / kWave; ++i) {
        const int e = lane + kWave * i, lo = e & 15, hi = e >> 4;
        v.r[i] = float2{pair_lut[2 * (lo * 16 + hi)], pair_lut[2 * (lo * 16 + hi) + 1]};  // (c[lo], c[hi])
    }
    return v;
}

template <int LAYOUT>
__device__ __forceinline__ void build_key_table(uint32_t *tbl, const LutRows &v, int lane) {
#pragma unroll
    for (int i = 0; i < 256 / kWave; ++i) {
        const int e = lane + kWave * i;
        const float c_lo = v.r[i].x, c_hi = v.r[i].y;
        const uint32_t p_lo = split_f16(c_lo), p_hi = split_f16(c_hi);
        tbl[2 * e] = (p_lo & 0xFFFFu) | (p_hi << 16);
        tbl[2 * e + 1] = (p_lo >> 16) | (p_hi & 0xFFFF0000u);
    }
}

// The rows i = w (mod nw) of the table (entries lane + 64 i), for a table that nw waves of a
// workgroup build together.
template <int LAYOUT>
__device__ __forceinline__ void build_key_table_rows(uint32_t *tbl, const LutRows &v, int lane, int w, int nw) {
#pragma unroll
    for (int i = 0; i < 256 / kWave; ++i) {
        if (i % nw != w)
            continue;
        const int e = lane + kWave * i;
        const uint32_t p_lo = split_f16(v.r[i].x), p_hi = split_f16(v.r[i].y);
        tbl[2 * e] = (p_lo & 0xFFFFu) | (p_hi << 16);
        tbl[2 * e + 1] = (p_lo >> 16) | (p_hi & 0xFFFF0000u);
    }
}

// 3-bit keys: entry e = a | b << 3 holds ((c_hi[a], c_hi[b]), (c_lo[a], c_lo[b])) -- the
// codes of a dim pair are 6 consecutive bits; one entry per lane (centroids [8]).
__device__ __forceinline__ void build_key_table3(uint32_t *tbl, const float *centroids, int lane) {
    const uint32_t pa = split_f16(centroids[lane & 7]), pb = split_f16(centroids[lane >> 3]);
    tbl[2 * lane] = (pa & 0xFFFFu) | (pb << 16);
    tbl[2 * lane + 1] = (pa >> 16) | (pb & 0xFFFF0000u);
}

// Per-lane byte offsets inside a KV block (fixed for a kernel instance); steps that are
// the same for every lane travel in the loads' scalar offsets.
struct LaneOffsets {
    uint32_t k;      // K bytes loaded by the lane: token 4g + n / 4, bytes 16 (n % 4) ..
    int kperm;       // 4 x the lane that loads the K bytes this lane needs (token n, bytes 16g ..)
    uint32_t v0;     // V dword n of token 4g; token 4g+i adds i * tok_stride
    uint32_t m;      // SoA: norm of the lane's first softmax token within its field array; AoS: its slot
    int tok_stride;  // bytes between consecutive tokens of one kv-head
    int mf;          // SoA: bytes between the three metadata arrays
    // SoA records of the presets, staged through LDS: where the lane writes its first 16
    // loaded bytes, reads its K bytes and its first V dword, and the byte shift that aligns a
    // 3-bit V dword read from two LDS dwords
    int kst, kld, vld, vsh;
    uint32_t k1, k2;  // FP8 keys: the second and third 16-byte chunks the lane loads
};

// Bytes per (token, kv-head) record: SoA data record / AoS slot; KF8: the FP8-key preset
// (128 K bytes | 64 V bytes, AoS + scale | zero).
// KB3: 3-bit keys, 4-bit values (turboquant_k3v4_nc): 48 K bytes | 64 V bytes (SoA), AoS
// K | norm | V | scale | zero = 118 bytes.
// V3 (with KB3): 3-bit values too (turboquant_3bit_nc): 48 K | 48 V bytes (SoA), AoS 102 bytes.
constexpr int kK3Bytes = kHeadDim * 3 / 8;
template <int LAYOUT, bool KF8, bool KB3 = false, bool V3 = false> constexpr int record_bytes() {
    return KF8   ? (LAYOUT == 0 ? kHeadDim + kHalfD : kHeadDim + kHalfD + 4)
           : KB3 ? (LAYOUT == 0 ? kK3Bytes + (V3 ? kK3Bytes : kHalfD) : kK3Bytes + (V3 ? kK3Bytes : kHalfD) + 6)
                 : (LAYOUT == 0 ? kSoaRecord : kAosSlot);
}
// Byte offset of the V codes in a record.
template <int LAYOUT, bool KF8, bool KB3 = false> constexpr int v_offset() {
    return KF8 ? kHeadDim : (KB3 ? kK3Bytes : kHalfD) + (LAYOUT == 0 ? 0 : 2);
}

// Record (t, h) of a block starts at t * pos + h * head: SoA pos = Hk * rec, head = rec;
// AoS position-major blocks [bs][Hk][slot] the same, head-major blocks [Hk][bs][slot] pos =
// slot, head = bs * slot (the caller passes the AoS strides).
template <int LAYOUT, int G, bool KF8 = false, bool KB3 = false, bool V3 = false>
__device__ __forceinline__ LaneOffsets lane_offsets(int n, int g, int kvh, int hk, int block_size, int pos,
                                                    int head) {
    constexpr int TPL = G / 4;
    const int st = 4 * g + TPL * (n / G);  // first softmax token of the lane
    const int rec = record_bytes<LAYOUT, KF8, KB3, V3>();
    if constexpr (LAYOUT == 0) {
        pos = hk * rec;
        head = rec;
    }
    LaneOffsets o;
    o.tok_stride = pos;
    // K is loaded coalesced (each 16-lane row reads 4 whole 64-byte K records) and then
    // permuted across lanes into the MFMA layout (lane (n, g) = token n, bytes 16g ..).
    // KB3 (3-bit keys): lane 16g + n loads 12 bytes, chunk (n & 3) of token 4g + (n >> 2), so
    // four consecutive lanes read one whole 48-byte K record; lane (n, g) then takes chunk g
    // of token n (the codes of dims 32g .. 32g+31) from lane 4n + g, as in the 4-bit case.
    o.k = (4 * g + (n >> 2)) * pos + kvh * head + (KB3 ? 12 : 16) * (n & 3);
    o.kperm = 4 * (16 * (n >> 2) + 4 * (n & 3) + g);
    // KF8: the second 64 K bytes are loaded the same way from o.k + 64
    // V3: the 3 bytes of dims 8n .. 8n+7 (a dword read; its fourth byte lies inside the
    // record or, for n = 15, is the next record's / the metadata's first byte, masked off)
    o.v0 = 4 * g * pos + kvh * head + v_offset<LAYOUT, KF8, KB3>() + (V3 ? 3 : 4) * n;
    if constexpr (KB3 && LAYOUT == 0) {
        // Whole records instead: lane l < 8C loads bytes 16c .. 16c+15 (c = l % C, C = rec / 16
        // lanes per record) of token l / C of the piece's first 8 tokens, and the same of token
        // 8 + l / C in a second load; a spare lane l >= 8C loads and stores what lane l - 8C
        // does (the same bytes to the same place).  In the LDS stage buffer record t sits at
        // t * rec.
        constexpr int R = record_bytes<LAYOUT, KF8, KB3, V3>(), C = R / 16;
        const int lane = 16 * g + n, l = lane % (8 * C);
        o.k = (l / C) * pos + kvh * head + 16 * (l % C);
        o.kst = (l / C) * R + 16 * (l % C);
        o.kld = n * R + 12 * g;
        o.vld = 4 * g * R + kK3Bytes + (V3 ? (3 * n) & ~3 : 4 * n);
        o.vsh = V3 ? (3 * n) & 3 : 0;
    }
    if constexpr (KF8 && LAYOUT == 0) {
        // FP8 keys, SoA: 192-byte records, 12 lanes each, 16 of them in three 16-byte-per-lane
        // loads (chunk q = 64 i + lane of load i is bytes 16 (q % 12) .. of token q / 12);
        // in the LDS stage buffer chunk q sits at 16 q
        constexpr int R = record_bytes<LAYOUT, KF8, KB3, V3>(), C = R / 16;
        const int lane = 16 * g + n;
        auto chunk = [&](int q) { return (uint32_t)((q / C) * pos + kvh * head + 16 * (q % C)); };
        o.k = chunk(lane);
        o.k1 = chunk(64 + lane);
        o.k2 = chunk(128 + lane);
        o.kst = 16 * lane;
        o.kld = n * R + 16 * g;
        o.vld = 4 * g * R + kHeadDim + 4 * n;
    }
    if (LAYOUT == 0) {
        // metadata fields: K norm, V scale, V zero (KF8: V scale, V zero)
        o.m = (kvh * (KF8 ? 2 : 3) * block_size + st) * 2;  // plus the piece's metadata offset (soffset)
        o.mf = block_size * 2;
    } else {
        o.m = st * pos + kvh * head;
        o.mf = 0;
    }
    return o;
}

// Raw K loads of one tile.
template <int LAYOUT> struct RawK;
template <> struct RawK<0> { uint4 k; };
template <> struct RawK<1> { uint4 k; };  // 2-byte aligned: gfx950 buffer loads take any byte offset
// Raw V + metadata loads of one tile.  SoA metadata of two consecutive tokens comes in
// one dword (TPL = 2); AoS: the norm in a 16-bit load per token, the adjacent scale and
// zero in one dword per token.
template <int LAYOUT, int TPL> struct RawV;
template <int TPL> struct RawV<0, TPL> {
    uint32_t v[4];
    uint32_t norm, scale, zero;
};
template <int TPL> struct RawV<1, TPL> {
    uint32_t v[4];
    uint32_t norm[TPL], scale_zero[TPL];
};

template <int LAYOUT>
__device__ __forceinline__ void issue_k(RawK<LAYOUT> &t, __amdgpu_buffer_rsrc_t rsrc, int doff,
                                        const LaneOffsets &o) {
    t.k = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, o.k, doff, 0));
}

// FP8 keys: the two 64-byte halves of the 128 K bytes, each loaded as a 4-bit K record is.
struct RawK8 {
    uint4 k, k2;
};
__device__ __forceinline__ void issue_k(RawK8 &t, __amdgpu_buffer_rsrc_t rsrc, int doff, const LaneOffsets &o) {
    t.k = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, o.k, doff, 0));
    t.k2 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, o.k + 64, doff, 0));
}

// 3-bit keys: 96 bits of one K record (after decode_k: the lane's dims 32g .. 32g+31, code d
// at bits 3(d - 32g)).
struct RawK3 {
    uint32_t w[3];
};
__device__ __forceinline__ void issue_k(RawK3 &t, __amdgpu_buffer_rsrc_t rsrc, int doff, const LaneOffsets &o) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b96(rsrc, o.k, doff, 0);
    t.w[0] = v[0];
    t.w[1] = v[1];
    t.w[2] = v[2];
}
__device__ __forceinline__ RawK3 decode_k(const RawK3 &t, const LaneOffsets &o) {
    RawK3 r;
#pragma unroll
    for (int i = 0; i < 3; ++i)
        r.w[i] = (uint32_t)__builtin_amdgcn_ds_bpermute(o.kperm, (int)t.w[i]);
    return r;
}

// 3-bit presets, SoA: the 112- or 96-byte records of a piece straddle 128-byte lines, which
// a K load and separate V loads would each request (2.6 / 2.5 line requests per record,
// against 1.75 / 1.5 when one load covers the whole record).  So the wave loads whole
// records, 16 bytes per lane (tokens 0-7, then 8-15), and hands them over through LDS.
struct RawRec {
    uint4 a, b;
};
__device__ __forceinline__ void issue_k(RawRec &t, __amdgpu_buffer_rsrc_t rsrc, int doff, const LaneOffsets &o) {
    t.a = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, o.k, doff, 0));
    t.b = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, o.k, doff + 8 * o.tok_stride, 0));
}
// The records into the stage buffer, then the lane's K bytes (token n, bytes 12g ..) and its
// V dwords (V dword n, or the 3-bit V bytes 3n .., of tokens 4g .. 4g+3) out of it.  One
// wave's LDS accesses run in program order, so the reads see these writes and the next
// piece's writes come after these reads.  The compiler barrier makes the compiler read
// what the other lanes wrote (its per-lane view would forward a lane's own earlier values).
template <int R, bool V3>
__device__ __forceinline__ RawK3 stage_records(const RawRec &t, uint8_t *buf, const LaneOffsets &o,
                                               uint32_t (&v)[4]) {
    *reinterpret_cast<uint4 *>(buf + o.kst) = t.a;
    *reinterpret_cast<uint4 *>(buf + o.kst + 8 * R) = t.b;
    asm volatile("" ::: "memory");
    const uint32_t *kp = reinterpret_cast<const uint32_t *>(buf + o.kld);
    RawK3 k;
#pragma unroll
    for (int i = 0; i < 3; ++i)
        k.w[i] = kp[i];
    const uint32_t *vp = reinterpret_cast<const uint32_t *>(buf + o.vld);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (V3)
            v[i] = __builtin_amdgcn_alignbyte(vp[i * R / 4 + 1], vp[i * R / 4], o.vsh);
        else
            v[i] = vp[i * R / 4];
    }
    return k;
}

// FP8 keys, SoA: the three loads of the staged records (see lane_offsets), then the lane's
// 32 K bytes (token n, bytes 16g .. of each 64-byte half) and its V dwords out of LDS, as
// stage_records does for the 3-bit presets.
struct RawRec3 {
    uint4 a, b, c;
};
__device__ __forceinline__ void issue_k(RawRec3 &t, __amdgpu_buffer_rsrc_t rsrc, int doff, const LaneOffsets &o) {
    t.a = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, o.k, doff, 0));
    t.b = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, o.k1, doff, 0));
    t.c = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, o.k2, doff, 0));
}

template <int LAYOUT, int TPL, bool KF8 = false, bool KB3 = false, bool V3 = false>
__device__ __forceinline__ void issue_v(RawV<LAYOUT, TPL> &t, __amdgpu_buffer_rsrc_t rsrc, int doff,
                                        int moff, const LaneOffsets &o) {
    if constexpr (KF8) {  // no K norm: fields V scale, V zero (SoA); scale | zero after V (AoS)
        if constexpr (LAYOUT == 1)  // SoA: the V codes come with the staged records
#pragma unroll
            for (int i = 0; i < 4; ++i)
                t.v[i] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, o.v0, doff + i * o.tok_stride, 0);
        if constexpr (LAYOUT == 0) {
            if constexpr (TPL == 1) {
                t.scale = __builtin_amdgcn_raw_buffer_load_b16(rsrc, o.m, moff, 0);
                t.zero = __builtin_amdgcn_raw_buffer_load_b16(rsrc, o.m, moff + o.mf, 0);
            } else {
                t.scale = __builtin_amdgcn_raw_buffer_load_b32(rsrc, o.m, moff, 0);
                t.zero = __builtin_amdgcn_raw_buffer_load_b32(rsrc, o.m, moff + o.mf, 0);
            }
            t.norm = 0x3C003C00u;  // f16 1.0 pair
        } else {
#pragma unroll
            for (int j = 0; j < TPL; ++j) {
                t.norm[j] = 0x3C00u;
                t.scale_zero[j] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, o.m + kHeadDim + kHalfD,
                                                                       doff + j * o.tok_stride, 0);
            }
        }
    } else if constexpr (LAYOUT == 0) {
        if constexpr (!KB3)  // 3-bit presets: the V codes come with the whole records
#pragma unroll
            for (int i = 0; i < 4; ++i)
                t.v[i] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, o.v0, doff + i * o.tok_stride, 0);
        if constexpr (TPL == 1) {
            t.norm = __builtin_amdgcn_raw_buffer_load_b16(rsrc, o.m, moff, 0);
            t.scale = __builtin_amdgcn_raw_buffer_load_b16(rsrc, o.m, moff + o.mf, 0);
            t.zero = __builtin_amdgcn_raw_buffer_load_b16(rsrc, o.m, moff + 2 * o.mf, 0);
        } else {
            t.norm = __builtin_amdgcn_raw_buffer_load_b32(rsrc, o.m, moff, 0);
            t.scale = __builtin_amdgcn_raw_buffer_load_b32(rsrc, o.m, moff + o.mf, 0);
            t.zero = __builtin_amdgcn_raw_buffer_load_b32(rsrc, o.m, moff + 2 * o.mf, 0);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            t.v[i] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, o.v0, doff + i * o.tok_stride, 0);
        constexpr int kKb = KB3 ? kK3Bytes : kHalfD;  // K bytes before the norm
        constexpr int kVb = V3 ? kK3Bytes : kHalfD;   // V bytes before scale | zero
#pragma unroll
        for (int j = 0; j < TPL; ++j) {
            t.norm[j] = __builtin_amdgcn_raw_buffer_load_b16(rsrc, o.m + kKb, doff + j * o.tok_stride, 0);
            t.scale_zero[j] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, o.m + kKb + 2 + kVb,
                                                                   doff + j * o.tok_stride, 0);
        }
    }
}

// The K bytes of lane (n, g) (token n, bytes 16g ..), gathered from the loading lanes.
template <int LAYOUT>
__device__ __forceinline__ uint4 decode_k(const RawK<LAYOUT> &t, const LaneOffsets &o) {
    const uint4 w = t.k;
    return uint4{(uint32_t)__builtin_amdgcn_ds_bpermute(o.kperm, (int)w.x),
                 (uint32_t)__builtin_amdgcn_ds_bpermute(o.kperm, (int)w.y),
                 (uint32_t)__builtin_amdgcn_ds_bpermute(o.kperm, (int)w.z),
                 (uint32_t)__builtin_amdgcn_ds_bpermute(o.kperm, (int)w.w)};
}

// FP8 keys: the lane's 32 K bytes (token n; bytes 16g .. 16g+15 of each 64-byte half).
struct K8 {
    uint4 a, b;
};
__device__ __forceinline__ K8 decode_k(const RawK8 &t, const LaneOffsets &o) {
    const RawK<0> h0{t.k}, h1{t.k2};
    return K8{decode_k<0>(h0, o), decode_k<0>(h1, o)};
}
__device__ __forceinline__ K8 stage_records(const RawRec3 &t, uint8_t *buf, const LaneOffsets &o, uint32_t (&v)[4]) {
    *reinterpret_cast<uint4 *>(buf + o.kst) = t.a;
    *reinterpret_cast<uint4 *>(buf + o.kst + 1024) = t.b;
    *reinterpret_cast<uint4 *>(buf + o.kst + 2048) = t.c;
    asm volatile("" ::: "memory");
    const K8 k{*reinterpret_cast<const uint4 *>(buf + o.kld), *reinterpret_cast<const uint4 *>(buf + o.kld + 64)};
    const uint32_t *vp = reinterpret_cast<const uint32_t *>(buf + o.vld);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        v[i] = vp[i * 48];  // token 4g + i: 192 bytes on
    return k;
}

// V dwords and metadata of one tile; metadata as f16 pairs (token j in half j).
struct TileV {
    uint32_t v[4];
    uint32_t norm, scale, zero;
};

template <int LAYOUT, int TPL>
__device__ __forceinline__ TileV decode_v(const RawV<LAYOUT, TPL> &t, const LaneOffsets &o) {
    TileV r;
    if constexpr (LAYOUT == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            r.v[i] = t.v[i];
        r.norm = t.norm;
        r.scale = t.scale;
        r.zero = t.zero;
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            r.v[i] = t.v[i];
        if constexpr (TPL == 1) {
            r.norm = t.norm[0];
            r.scale = t.scale_zero[0] & 0xFFFFu;
            r.zero = t.scale_zero[0] >> 16;
        } else {
            r.norm = (t.norm[0] & 0xFFFFu) | (t.norm[1] << 16);
            r.scale = __builtin_amdgcn_perm(t.scale_zero[1], t.scale_zero[0], 0x05040100u);
            r.zero = __builtin_amdgcn_perm(t.scale_zero[1], t.scale_zero[0], 0x07060302u);
        }
    }
    return r;
}

// a / b for a >= 0, b > 0 (uniform): a shift when b is a power of two, as split counts,
// split lengths and waves per sequence usually are, else the division
__device__ __forceinline__ int div_pos(int a, int b) {
    if ((b & (b - 1)) == 0)
        return a >> __builtin_ctz((unsigned)b);
    return a / b;
}

// Waves of one kv-head dealt to the sequences.  The grid gives every kv-head nw * B
// waves (wave x = wid + nw * b), a number fixed by the shapes alone.  A sequence with live
// splits gets one wave plus a share of the other nw * B - n_live in proportion to its
// estimated stream length (prefix rounding: the shares sum to at most that many), and at
// most one wave per live split; each wave then takes a run of its sequence's live splits
// (k waves over `live` splits: the first live % k runs one split longer).  Every wave of the
// kv-head computes the same deal from seq_lens, so ragged batches keep the waves about
// equally busy; equal lengths give every sequence nw waves (taken without the arithmetic);
// batches of at most 64 sequences also pair heavy runs with light ones on each SIMD
// (deal_ranked).
struct Deal {
    int b, wid, nw;  // b < 0: the deal leaves this wave without work
    int len;         // seq_lens[b], as the deal read it
};

// Live splits and estimated stream positions of a sequence of len tokens (sequence bb, 0
// past the batch): each split's tiles (one more when it straddles a tile edge), as the
// stream pads them.
struct SeqLoad {
    int live;
    uint32_t est;
    int len;
    int per;  // estimated positions per split
};
__device__ __forceinline__ SeqLoad sequence_load_len(int len, int S) {
    len = max(len, 0);
    const int split_len = div_pos(len + S - 1, S);
    const int live = split_len > 0 ? (len + split_len - 1) / split_len : 0;
    const int per = ((split_len + 15) >> 4) + 1;
    return SeqLoad{live, (uint32_t)live * (uint32_t)per, len, per};
}
__device__ __forceinline__ SeqLoad sequence_load(const int32_t *__restrict__ seq_lens, int B, int S, int bb) {
    return sequence_load_len(bb < B ? seq_lens[bb] : 0, S);
}

// Inclusive prefix sum over the wave's 64 lanes: shifts within each 16-lane row, then the
// row totals broadcast into the rows after them.
__device__ __forceinline__ uint32_t wave_scan(uint32_t v) {
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, true);   // row_shr:1
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, true);   // row_shr:2
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, true);   // row_shr:4
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, true);   // row_shr:8
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false);  // row_bcast:15 -> rows 1, 3
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false);  // row_bcast:31 -> rows 2, 3
    return v;
}

// Stream totals stay far below 2^32: a position covers 16 tokens of one kv-head.
// Lane-wide sum and max (the value of lane 63 after an inclusive scan; max for values >= 0).
__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_readlane((int)wave_scan(v), kWave - 1);
}
__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, true));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, true));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, true));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, true));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, kWave - 1);
}

// Batches of at most 64 sequences (one lane each): the waves of the deal, each a run of its
// sequence's splits (k waves over `live` splits: the first live % k runs one split longer),
// are ranked by estimated stream positions, heaviest first (ties: by sequence, then run).
// Grid waves x and x + nw*B/2 share a SIMD when the grid is one round of the device at two
// waves per SIMD (workgroups i and i + half are dispatched to one SIMD), so they take ranks p
// and nw*B - 1 - p: a heavy run shares its SIMD with a light one.  The rank-p wave is found
// by bisection on its load (lane-wide counts of the waves at least that heavy), then by its
// place among the waves of exactly that load.  Any x -> p bijection keeps the deal exact.
// lane_len: seq_lens[lane] (0 past the batch), read by the caller.
__device__ Deal deal_ranked(int lane_len, int B, int S, int nw, int x, int lane) {
    const SeqLoad q = sequence_load_len(lane_len, S);
    const uint32_t est_total = wave_sum(q.est);
    const int n_live = __builtin_popcountll(__ballot(q.live > 0));
    // spare waves before prefix pre: floor(pre * spare / total) with one fp32 ratio -- monotone
    // in pre and at most `spare` at the total, the same on every wave (all the deal needs)
    const float ratio = est_total > 0 ? (float)((int64_t)nw * B - n_live) / (float)est_total : 0.f;
    auto cut = [&](uint32_t pre) { return (int)floorf((float)pre * ratio); };
    const uint32_t est_out = wave_scan(q.est);
    const int k = q.live > 0 ? min(1 + cut(est_out) - cut(est_out - q.est), q.live) : 0;
    const int per = q.live > 0 ? q.per : 0;  // positions per split
    // live / k and live % k: an fp32 quotient is within 1 of it for live below 2^22 (live <= S),
    // so one correction step makes it exact
    int qd = 0, r = 0;
    if (k > 0) {
        qd = (int)((float)q.live * __builtin_amdgcn_rcpf((float)k));
        r = q.live - qd * k;
        if (r < 0) {
            --qd;
            r += k;
        } else if (r >= k) {
            ++qd;
            r -= k;
        }
    }
    const uint32_t l_hi = (uint32_t)((qd + 1) * per), l_lo = (uint32_t)(qd * per);
    const int n_hi = r, n_lo = k - r;  // runs of qd + 1 and of qd splits
    const int T = nw * B;
    const int p = (T % 2 == 0 && x >= T / 2) ? 3 * T / 2 - 1 - x : x;
    if ((uint32_t)p >= wave_sum((uint32_t)k))
        return Deal{-1, 0, 0, -1};
    auto count_ge = [&](uint32_t t) {
        return wave_sum((uint32_t)((n_hi > 0 && l_hi >= t ? n_hi : 0) + (n_lo > 0 && l_lo >= t ? n_lo : 0)));
    };
    // the load of rank p: the largest t with more than p waves at least that heavy
    uint32_t lo = 0, hi = wave_max(n_hi > 0 ? l_hi : l_lo) + 1;
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) / 2;
        if (count_ge(mid) > (uint32_t)p)
            lo = mid;
        else
            hi = mid;
    }
    const int idx = p - (int)count_ge(lo + 1);
    const bool hi_in = n_hi > 0 && l_hi == lo;
    const int in_b = hi_in ? n_hi : (n_lo > 0 && l_lo == lo ? n_lo : 0);
    const int incl = (int)wave_scan((uint32_t)in_b), excl = incl - in_b;
    const uint64_t hit = __ballot(in_b > 0 && idx >= excl && idx < incl);
    const int sq = __builtin_ctzll(hit);
    const int j0 = idx - __builtin_amdgcn_readlane(excl, sq);
    const int j = __builtin_amdgcn_readlane(hi_in ? 1 : 0, sq) ? j0 : __builtin_amdgcn_readlane(r, sq) + j0;
    return Deal{sq, j, __builtin_amdgcn_readlane(k, sq), __builtin_amdgcn_readlane(q.len, sq)};
}

__device__ Deal deal_waves(const int32_t *__restrict__ seq_lens, int B, int S, int nw, int x, int lane) {
    // equal lengths: every sequence keeps its nw waves, as the deal would give them
    const int len0 = seq_lens[0];
    bool equal = true;
    int lane_len = 0;  // seq_lens[lane] (0 past the batch): the first 64 lengths, read once
    for (int c0 = 0; c0 < B; c0 += kWave) {
        const int bb = c0 + lane;
        const int len = bb < B ? seq_lens[bb] : len0;
        if (c0 == 0)
            lane_len = bb < B ? len : 0;
        equal = equal && __ballot(len != len0) == 0;
    }
    if (equal)
        return Deal{x / nw, x % nw, nw, len0};
    if (B <= kWave)
        return deal_ranked(lane_len, B, S, nw, x, lane);
    const SeqLoad first = sequence_load_len(lane_len, S);
    uint32_t est_total = 0;
    int n_live = 0;
    for (int c0 = 0; c0 < B; c0 += kWave) {
        const SeqLoad q = c0 == 0 ? first : sequence_load(seq_lens, B, S, c0 + lane);
        est_total += (uint32_t)__builtin_amdgcn_readlane((int)wave_scan(q.est), kWave - 1);
        n_live += __builtin_popcountll(__ballot(q.live > 0));
    }
    const double spare = (double)((int64_t)nw * B - n_live);
    // spare waves dealt to the sequences before prefix p: floor(spare * p / total), exact in
    // double (the quotient of integers below 2^53 lands on an integer only when it is one)
    auto cut = [&](uint32_t p) { return est_total > 0 ? (int)floor(spare * (double)p / (double)est_total) : 0; };
    uint32_t est_carry = 0;
    int wave_carry = 0;
    for (int c0 = 0; c0 < B; c0 += kWave) {
        const SeqLoad q = c0 == 0 ? first : sequence_load(seq_lens, B, S, c0 + lane);
        const uint32_t est_out = est_carry + wave_scan(q.est);
        const int mine = q.live > 0 ? min(1 + cut(est_out) - cut(est_out - q.est), q.live) : 0;
        const int w_out = wave_carry + (int)wave_scan((uint32_t)mine);
        const int w_in = w_out - mine;
        const uint64_t hit = __ballot(x >= w_in && x < w_out);
        if (hit) {
            const int l = __builtin_ctzll(hit);
            return Deal{c0 + l, x - __builtin_amdgcn_readlane(w_in, l), __builtin_amdgcn_readlane(mine, l),
                        __builtin_amdgcn_readlane(q.len, l)};
        }
        est_carry = (uint32_t)__builtin_amdgcn_readlane((int)est_out, kWave - 1);
        wave_carry = __builtin_amdgcn_readlane(w_out, kWave - 1);
    }
    return Deal{-1, 0, 0, -1};
}

// Running softmax state of a lane: the shared max of its head (as -m, exp2 domain;
// +FLT_MAX = "no token yet"), the lane's own partial sums.
struct State {
    float negm, l, z;
    float pend;  // rescale of the accumulators still owed for the lane's head (applied by the next PV stage)
};

// Lane constants of the token selection / operand packing.
struct LaneConst {
    int n, g;
    bool tok_bit0, tok_bit1;  // G = 4: register index n / 4 of the lane's token
    bool upper;               // n >= 8: rows / columns of the lo part
    uint32_t part_sel;        // v_perm selector of the lane's part (hi / lo halves)
};

// q as B operands of the 8 QK^T MFMAs of a tile.  MFMA m covers the lane's code bytes
// 2m, 2m+1 (dims d = 32g + 4m .. +3); its A slots are (c_hi, c_hi, c_lo, c_lo) of byte 2m
// then of byte 2m+1, so bq[m] = (Q(2m), Q(2m), Q(2m+1), Q(2m+1)) with Q(b) the f16 pair
// q_part(n)[head kvh*G + (n & (G-1))][32g + 2b, 32g + 2b + 1].
// kf8: the lane-local dims of the FP8-key layout (dims 16g + 4m, m < 4; 64 + 16g + 4(m - 4)).
__device__ __forceinline__ void load_q_rows(float4 (&qx)[8], const float *__restrict__ q_rot, int64_t head_row,
                                            int g, bool kf8 = false) {
    const float *qr = q_rot + head_row * kHeadDim;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const int d = kf8 ? (m < 4 ? 16 * g + 4 * m : 64 + 16 * g + 4 * (m - 4)) : 32 * g + 4 * m;
        qx[m] = *reinterpret_cast<const float4 *>(qr + d);
    }
}
// A q row whose largest |q * scale| reaches 2^15 is first scaled by the power of two 2^e
// (e < 0) that puts it in [2^14, 2^15), inside the f16 range of the hi part; the returned
// 2^-e (1 for every other row, so their scores are unchanged bit for bit) multiplies the
// lane's dots.  The row's four lanes n, n + 16, n + 32, n + 48 share the maximum.
__device__ __forceinline__ float q_operands(half8 (&bq)[8], const float4 (&qx)[8], int n, float scale) {
    float amax = 0.f;
#pragma unroll
    for (int m = 0; m < 8; ++m)
        amax = fmaxf(fmaxf(fmaxf(amax, fabsf(qx[m].x)), fmaxf(fabsf(qx[m].y), fabsf(qx[m].z))), fabsf(qx[m].w));
    amax = rot_row_max(amax) * scale;
    const int e = (amax >= 32768.f && amax < __builtin_inff()) ? 15 - __builtin_amdgcn_frexp_expf(amax) : 0;
    const float rs = __builtin_ldexpf(scale, e);
    // the lane's part (hi for n < 8, lo for n >= 8) of two split values, packed
    const uint32_t sel = n >= 8 ? 0x07060302u : 0x05040100u;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const float4 x = qx[m];
        const uint32_t s0 = split_f16(x.x * rs), s1 = split_f16(x.y * rs);
        const uint32_t s2 = split_f16(x.z * rs), s3 = split_f16(x.w * rs);
        const uint32_t w0 = __builtin_amdgcn_perm(s1, s0, sel);
        const uint32_t w1 = __builtin_amdgcn_perm(s3, s2, sel);
        bq[m] = as_half8(w0, w0, w1, w1);
    }
    return __builtin_ldexpf(1.f, -e);
}

// K-table entries of one tile's 16 code bytes (dims 32g + 2b, 32g + 2b + 1 for byte b),
// read from LDS at the top of a stage so that their latency is covered by the softmax
// that runs meanwhile; AoS also sums the lane's share of ||c[idx]||^2.
struct KOps {
    uint2 e[16];
    float csq;
};

template <int LAYOUT>
__device__ __forceinline__ KOps lookup_tile(const uint4 &k, const uint32_t *ktab) {
    KOps r;
    const uint32_t kw[4] = {k.x, k.y, k.z, k.w};
    const uint2 *t2 = reinterpret_cast<const uint2 *>(ktab);
#pragma unroll
    for (int b = 0; b < 16; ++b)
        r.e[b] = t2[(kw[b >> 2] >> (8 * (b & 3))) & 0xFFu];
    r.csq = 0.f;
    if constexpr (LAYOUT == 1) {
        // c_lo^2 + c_hi^2 of every byte from its own entry: c = h + l (f16 parts), so
        // sum c^2 = sum h.h + 2 sum h.l (+ l.l, below fp32 rounding); f16 products are exact
        float hh = 0.f, hl = 0.f;
#pragma unroll
        for (int b = 0; b < 16; ++b) {
            const auto h = __builtin_bit_cast(__fp16 __attribute__((ext_vector_type(2))), r.e[b].x);
            const auto l = __builtin_bit_cast(__fp16 __attribute__((ext_vector_type(2))), r.e[b].y);
            hh = __builtin_amdgcn_fdot2(h, h, hh, false);
            hl = __builtin_amdgcn_fdot2(h, l, hl, false);
        }
        r.csq = fmaf(2.f, hl, hh);
    }
    return r;
}

// FP8 keys: entry b = the f16 pair of the lane's K bytes 2b, 2b+1 (E4M3 -> f16 is exact), lo
// part 0.  Lane-local dim i is dim 16g + i (i < 16) or 64 + 16g + i - 16 (the two halves).
__device__ __forceinline__ KOps lookup_tile(const K8 &k, const uint32_t *) {
    KOps r;
    const uint32_t kw[8] = {k.a.x, k.a.y, k.a.z, k.a.w, k.b.x, k.b.y, k.b.z, k.b.w};
#pragma unroll
    for (int w = 0; w < 8; ++w) {
        const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)kw[w], false);  // bytes 0, 1
        const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)kw[w], true);   // bytes 2, 3
        r.e[2 * w].x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo[0], lo[1]));
        r.e[2 * w + 1].x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(hi[0], hi[1]));
        r.e[2 * w].y = r.e[2 * w + 1].y = 0u;
    }
    r.csq = 0.f;
    return r;
}

// 3-bit keys: entry b = the table entry of the lane's dims 2b, 2b+1 (bits 6b .. 6b+5 of its
// 96 bits; pairs 5 and 10 straddle a word boundary); AoS sums ||c||^2 as the 4-bit path.
template <int LAYOUT>
__device__ __forceinline__ KOps lookup_tile(const RawK3 &k, const uint32_t *ktab) {
    KOps r;
    const uint2 *t2 = reinterpret_cast<const uint2 *>(ktab);
#pragma unroll
    for (int b = 0; b < 16; ++b) {
        const int bit = 6 * b, wi = bit >> 5, sh = bit & 31;
        uint32_t v = k.w[wi] >> sh;
        if (sh > 26)
            v |= k.w[wi + 1] << (32 - sh);
        r.e[b] = t2[v & 63u];
    }
    r.csq = 0.f;
    if constexpr (LAYOUT == 1) {
        float hh = 0.f, hl = 0.f;
#pragma unroll
        for (int b = 0; b < 16; ++b) {
            const auto h = __builtin_bit_cast(__fp16 __attribute__((ext_vector_type(2))), r.e[b].x);
            const auto l = __builtin_bit_cast(__fp16 __attribute__((ext_vector_type(2))), r.e[b].y);
            hh = __builtin_amdgcn_fdot2(h, h, hh, false);
            hl = __builtin_amdgcn_fdot2(h, l, hl, false);
        }
        r.csq = fmaf(2.f, hl, hh);
    }
    return r;
}

__device__ __forceinline__ half8 k_operand(const KOps &k, int m) {
    return as_half8(k.e[2 * m].x, k.e[2 * m].y, k.e[2 * m + 1].x, k.e[2 * m + 1].y);
}

// QK^T of one tile from its looked-up entries: 8 MFMAs in two accumulation chains.
__device__ __forceinline__ floatx4 qk_tile(const KOps &k, const half8 (&bq)[8]) {
    floatx4 h = {0.f, 0.f, 0.f, 0.f}, l = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 8; m += 2) {
        h = mfma(k_operand(k, m), bq[m], h);
        l = mfma(k_operand(k, m + 1), bq[m + 1], l);
    }
    return h + l;
}

// PV of a pair of tiles (A operand aw, V dwords va / vb of tokens 4g .. 4g+3) interleaved
// with QK^T of the next tile.  V codes enter as f16 denormal bit patterns (integer k <->
// k * 2^-24), placed in the top bits of the 10-bit significand: the matrix core aligns a
// product with a denormal factor at the denormal exponent, so every leading zero of the
// significand would cut that product's share of the truncated in-lane sum.
// Accumulator 2m takes the even dim's codes (low nibble << 6, units 2^-18), accumulator
// 2m + 1 the whole bytes (byte << 2, units 2^-22: lo + 16 * hi); the odd dim is recovered as
// (16 acc[2m+1] - acc[2m]) * 2^14 when the split's rows are written.  V3 (3-bit values, dims
// 8n .. 8n+7 at bits 3(d - 8n) of the lane's dword): accumulator 2m takes the even dim's
// codes, 2m + 1 the odd dim's, each a 3-bit field << 7 (units 2^-17).
constexpr float kVUnitEven = 262144.0f;  // 2^18: 4-bit low nibble << 6
constexpr float kVUnitOdd = 16384.0f;    // 2^14: (16 * (byte << 2) - (nibble << 6)) units
constexpr float kVUnit3 = 131072.0f;     // 2^17: 3-bit code << 7
template <bool V3 = false>
__device__ __forceinline__ floatx4 pv_qk(floatx4 (&acc)[8], const uint32_t (&aw)[4], const uint32_t (&va)[4],
                                         const uint32_t (&vb)[4], const KOps &k, const half8 (&bq)[8]) {
    const half8 a = as_half8(aw[0], aw[1], aw[2], aw[3]);
    floatx4 h = {0.f, 0.f, 0.f, 0.f}, l = {0.f, 0.f, 0.f, 0.f};
    if constexpr (V3) {
        // Two tokens' dwords x, y -> window w: (x bits 8w .. 8w+15) | (y bits 8w .. 8w+15) << 16,
        // one v_perm; dims 0-4 of the lane lie in window 0, dims 5-7 in window 1.  A dim's code
        // pair then sits at the same bit of both halves, and one shift and one mask move it to
        // (code_x << 7, code_y << 7): a shift of d <= 7 bits carries the low half's upper bits
        // only below bit 7 of the high half, a right shift of |d| <= 6 the high half's lower
        // bits only above bit 9 of the low half, and the mask clears both.
        uint32_t win[2][4];
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const uint32_t sel = w == 0 ? 0x05040100u : 0x06050201u;
            win[w][0] = __builtin_amdgcn_perm(va[1], va[0], sel);
            win[w][1] = __builtin_amdgcn_perm(va[3], va[2], sel);
            win[w][2] = __builtin_amdgcn_perm(vb[1], vb[0], sel);
            win[w][3] = __builtin_amdgcn_perm(vb[3], vb[2], sel);
        }
        auto codes = [&](int j, int i) {
            const int w = j < 5 ? 0 : 1, d = 7 - (3 * j - 8 * w);
            return (d >= 0 ? win[w][i] << d : win[w][i] >> -d) & 0x03800380u;
        };
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int je = 2 * m, jo = 2 * m + 1;
            h = mfma(k_operand(k, 2 * m), bq[2 * m], h);
            acc[2 * m] = mfma(a, as_half8(codes(je, 0), codes(je, 1), codes(je, 2), codes(je, 3)), acc[2 * m]);
            l = mfma(k_operand(k, 2 * m + 1), bq[2 * m + 1], l);
            acc[2 * m + 1] = mfma(a, as_half8(codes(jo, 0), codes(jo, 1), codes(jo, 2), codes(jo, 3)), acc[2 * m + 1]);
        }
        return h + l;
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        // byte m (dims 8n + 2m, 8n + 2m + 1) of two tokens' dwords -> (byte, 0, byte, 0)
        const uint32_t sel = (uint32_t)m | 0x0C00u | ((uint32_t)(4 + m) << 16) | 0x0C000000u;
        const uint32_t p0 = __builtin_amdgcn_perm(va[1], va[0], sel), p1 = __builtin_amdgcn_perm(va[3], va[2], sel);
        const uint32_t p2 = __builtin_amdgcn_perm(vb[1], vb[0], sel), p3 = __builtin_amdgcn_perm(vb[3], vb[2], sel);
        h = mfma(k_operand(k, 2 * m), bq[2 * m], h);
        acc[2 * m] = mfma(a, as_half8((p0 << 6) & 0x03C003C0u, (p1 << 6) & 0x03C003C0u, (p2 << 6) & 0x03C003C0u,
                                      (p3 << 6) & 0x03C003C0u), acc[2 * m]);
        l = mfma(k_operand(k, 2 * m + 1), bq[2 * m + 1], l);
        acc[2 * m + 1] = mfma(a, as_half8(p0 << 2, p1 << 2, p2 << 2, p3 << 2), acc[2 * m + 1]);
    }
    return h + l;
}

// Full dot of the lane's TPL softmax tokens from the QK^T accumulator (+ column n ^ 8).
template <int G>
__device__ __forceinline__ void lane_dots(const floatx4 &acc, const LaneConst &lc, float (&dot)[G / 4]) {
    float d[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        d[i] = acc[i] + dppf<kRor8>(acc[i]);
    if constexpr (G == 4) {
        const float lo = lc.tok_bit0 ? d[1] : d[0];
        const float hi = lc.tok_bit0 ? d[3] : d[2];
        dot[0] = lc.tok_bit1 ? hi : lo;
    } else {
        dot[0] = lc.upper ? d[2] : d[0];
        dot[1] = lc.upper ? d[3] : d[1];
    }
}

// Max over the lanes of one head (G = 4: lanes n = h mod 4 of all rows; G = 8: n = h mod 8).
template <int G> __device__ __forceinline__ float head_max(float x) {
    x = max_score(x, dppf<kRor8>(x));
    if constexpr (G == 4)
        x = max_score(x, dppf<kRor4>(x));
    return max_xor16(max_xor32(x));
}
template <int G> __device__ __forceinline__ float head_sum(float x) {
    x += dppf<kRor8>(x);
    if constexpr (G == 4)
        x += dppf<kRor4>(x);
    return sum_xor16(sum_xor32(x));
}

// w * a of a pending PV A-operand dword (two tokens' w as f16 parts of the lane's row;
// the other part sits in lane n ^ 8 of the same row), split again into the lane's part.
__device__ __forceinline__ uint32_t rescale_pending(uint32_t d, float a, bool upper) {
    const uint32_t other = dpp<kRor8>(d);
    const uint32_t hi = upper ? other : d, lo = upper ? d : other;
    const uint32_t s0 = split_f16((half_at(hi, 0) + half_at(lo, 0)) * a);
    const uint32_t s1 = split_f16((half_at(hi, 1) + half_at(lo, 1)) * a);
    return upper ? ((s0 >> 16) | (s1 & 0xFFFF0000u)) : ((s0 & 0xFFFFu) | (s1 << 16));
}

// Softmax of one tile -> the lane's two A-operand dwords d0 / d1 of the PV (tokens 4g ..
// 4g+3 of the lane's head row, in its part).  dots: the lane's token dots; norm_f:
// per-token score factors; valid: token inside the split (only boundary tiles have
// invalid ones).  A max change on the first tile of a pair only records the factor the
// accumulators owe (st.pend); the second tile (SECOND) applies it, with its own, before
// the pair's PV, and rescales the first tile's dwords p0 / p1, still waiting for that PV.
// Only the second tile's rare branch touches the accumulators, so the common path keeps
// them in place.
template <int G, bool SECOND>
__device__ __forceinline__ void softmax_tile(const float (&dot)[G / 4], const float (&norm_f)[G / 4],
                                             const TileV &t, State &st, floatx4 (&acc)[8],
                                             const LaneConst &lc, bool boundary,
                                             const bool (&valid)[G / 4], uint32_t &p0, uint32_t &p1,
                                             uint32_t &d0, uint32_t &d1) {
    constexpr int TPL = G / 4;
    float s2[TPL], vscale[TPL], vzero[TPL];
    bool need = false;
#pragma unroll
    for (int j = 0; j < TPL; ++j) {
        s2[j] = fmaf(dot[j], norm_f[j], st.negm);  // score - m
        vscale[j] = half_at(t.scale, j);
        vzero[j] = half_at(t.zero, j);
    }
    if (__builtin_expect(boundary, 0)) {
        // tokens outside the split: p = 0, and their (unwritten, possibly non-finite) V
        // scale and zero must not reach p * scale, p * zero
#pragma unroll
        for (int j = 0; j < TPL; ++j) {
            s2[j] = valid[j] ? s2[j] : -INFINITY;
            vscale[j] = valid[j] ? vscale[j] : 0.f;
            vzero[j] = valid[j] ? vzero[j] : 0.f;
        }
    }
#pragma unroll
    for (int j = 0; j < TPL; ++j)
        need |= s2[j] > kRescaleLogX;
    if constexpr (SECOND)
        need |= st.pend != 1.f;
    if (__builtin_expect(__any(need), 0)) {
        // new head max from the exact scores (s2 is inexact while -m = FLT_MAX)
        float sn[TPL];
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < TPL; ++j) {
            sn[j] = dot[j] * norm_f[j];
            if (boundary)
                sn[j] = valid[j] ? sn[j] : -INFINITY;
            mx = max_score(mx, sn[j]);
        }
        mx = head_max<G>(mx);
        const float negm_new = (mx + st.negm > kRescaleLogX) ? -mx : st.negm;
        // exp2(m_old - m_new): 1 for heads that keep their max, 0 after a split start
        const float alpha = __builtin_amdgcn_exp2f(negm_new - st.negm);
        st.l *= alpha;
        st.z *= alpha;
        if constexpr (SECOND) {
            const float owed = alpha * st.pend;
            st.pend = 1.f;
            float ah[4];
            if constexpr (G == 4) {
                ah[0] = quad_bcast<0>(owed);  // lane 4q + r holds head r
                ah[1] = quad_bcast<1>(owed);
                ah[2] = quad_bcast<2>(owed);
                ah[3] = quad_bcast<3>(owed);
            } else {
                // accumulator register r of lane group g = head r + 4 (g & 1); row 0 lane h
                // holds head h
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    ah[r] = __shfl(owed, r + 4 * (lc.g & 1), kWave);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j)
                acc[j] *= floatx4{ah[0], ah[1], ah[2], ah[3]};
            p0 = rescale_pending(p0, alpha, lc.upper);
            p1 = rescale_pending(p1, alpha, lc.upper);
        } else if (st.negm != __FLT_MAX__) {
            // (a split's first tile finds the accumulators already cleared: nothing owed)
            st.pend *= alpha;
        }
        st.negm = negm_new;
#pragma unroll
        for (int j = 0; j < TPL; ++j)
            s2[j] = sn[j] + negm_new;
    }
    uint32_t y[TPL];
#pragma unroll
    for (int j = 0; j < TPL; ++j) {
        const float p = __builtin_amdgcn_exp2f(s2[j]);
        st.l += p;
        st.z = fmaf(p, vzero[j], st.z);
        y[j] = split_f16(p * vscale[j]);
    }
    uint32_t P, Q;
    if constexpr (G == 4) {
        // lane n owns token n / 4; lanes n + 4, n + 8, n + 12 own the next ones (mod 4)
        const uint32_t x1 = dpp<kRor12>(y[0]), x2 = dpp<kRor8>(y[0]), x3 = dpp<kRor4>(y[0]);
        P = __builtin_amdgcn_perm(x1, y[0], lc.part_sel);
        Q = __builtin_amdgcn_perm(x3, x2, lc.part_sel);
    } else {
        // lane n owns tokens 2 (n / 8) + {0, 1}; lane n ^ 8 owns the other two
        const uint32_t z0 = dpp<kRor8>(y[0]), z1 = dpp<kRor8>(y[1]);
        P = __builtin_amdgcn_perm(y[1], y[0], lc.part_sel);
        Q = __builtin_amdgcn_perm(z1, z0, lc.part_sel);
    }
    // rows 0..7 own tokens (0, 1) in P; rows 8..15 own tokens (2, 3) in P
    d0 = lc.upper ? Q : P;
    d1 = lc.upper ? P : Q;
}

// Split rows go to mid_o through an LDS image of the wave's part of it: for head h the
// image holds the rows of up to Cap::splits consecutive splits back to back (129
// floats each, as in mid_o), and one flush writes each head's run with contiguous 16-byte
// stores.  A few long write runs instead of one 516-byte row per head and split keep the
// HBM writes from breaking up the read stream.
// The image takes what the K-code table leaves of a wave's share of the CU's 160 KB LDS
// at WPE waves per SIMD.
// RESERVED: the kernel's other LDS (K table, record stage buffer)
template <int LAYOUT, int G, int WPE, int RESERVED> struct SpanCap {
    static constexpr int bytes = 160 * 1024 / (4 * WPE) - RESERVED;
    static constexpr int row_floats = kHeadDim + 1;
    static constexpr int splits = (bytes / 4 / G) / row_floats;         // rows per head
    static constexpr int head_floats = (splits * row_floats + 3) & ~3;  // 16 B aligned
    static constexpr int floats = G * head_floats;
    static_assert(splits >= 1 && floats * 4 <= bytes, "LDS image does not fit");
};

// LSE of a split, (m + log2 l) * ln 2 with the scores in log2 units.  l >= 1: the running
// max is only ever set to the score of one of the split's tokens (whose p is then 1), or
// the caller passes 1 for a split without valid tokens; so the hardware log2 sees a normal
// number (1 ulp).
__device__ __forceinline__ float lse_of(float negm, float l) {
    return (__builtin_amdgcn_logf(l) - negm) * kLn2;
}

// Output rows of a finished split held by this lane: heads h0 .. h0 + G/4 - 1, dims 8n ..
// 8n + 7 each, from the hi and lo halves of the PV sums (lanes l and l ^ 32, summed with
// rs_xor32), plus the head's softmax sum (safe_l, 1 for an empty split).
// G = 8: lane group g ends with heads hA = 2 (g >> 1) + 4 (g & 1) and hA + 1 (register
// elements 0 / 2 and 1 / 3).  G = 4: only lane groups 0 and 2 hold usable rows (rows 0..3
// hi, 8..11 lo; the A rows 4..7 and 12..15 carry the same heads with their tokens in a
// rotated slot order, so those sums are discarded).  A v_permlane16_swap of elements 0 and
// 1 (2 and 3) moves group 0's element 1 (3) into group 1 and group 2's into group 3, and
// each lane group then finishes one head, g: half the arithmetic of taking two heads in
// groups 0 and 2 while groups 1 and 3 idle.
template <int G, bool V3>
__device__ __forceinline__ void finish_rows(const State &st, const floatx4 (&acc)[8], const LaneConst &lc, int &h0,
                                            float (&o)[G / 4][8], float &safe_l) {
    const float lt = head_sum<G>(st.l);
    const float zt = head_sum<G>(st.z);
    safe_l = lt > 0.f ? lt : 1.f;
    // accumulator 2m + 1 holds the whole bytes (even + 16 * odd), or (V3) the odd dim's
    // codes, in the units of pv_qk; every row holds the totals of head h in lanes n = h (mod G)
    auto dims = [](float x, float y, float z, float inv, float &even, float &odd) {
        if constexpr (V3) {
            even = fmaf(x, kVUnit3, z) * inv;
            odd = fmaf(y, kVUnit3, z) * inv;
        } else {
            even = fmaf(x, kVUnitEven, z) * inv;
            odd = fmaf(fmaf(y, 16.f, -x), kVUnitOdd, z) * inv;
        }
    };
    if constexpr (G == 4) {
        h0 = lc.g;
        // rows 0 and 2 of the result keep element 2k of groups 0 and 2, rows 1 and 3 receive
        // element 2k + 1 of groups 0 and 2
        auto head_rows = [](float ek, float ek1) {
            return bitsf(__builtin_amdgcn_permlane16_swap(fbits(ek), fbits(ek1), false, false)[0]);
        };
        const float inv = __builtin_amdgcn_rcpf(__shfl(safe_l, h0, kWave));
        const float z = __shfl(zt, h0, kWave);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const floatx4 &e = acc[2 * m], &w = acc[2 * m + 1];
            const float x = rs_xor32(head_rows(e[0], e[1]), head_rows(e[2], e[3]));
            const float y = rs_xor32(head_rows(w[0], w[1]), head_rows(w[2], w[3]));
            dims(x, y, z, inv, o[0][2 * m], o[0][2 * m + 1]);
        }
    } else {
        h0 = 2 * (lc.g >> 1) + 4 * (lc.g & 1);
        const float inv_a = __builtin_amdgcn_rcpf(__shfl(safe_l, h0, kWave));
        const float inv_b = __builtin_amdgcn_rcpf(__shfl(safe_l, h0 + 1, kWave));
        const float z_a = __shfl(zt, h0, kWave), z_b = __shfl(zt, h0 + 1, kWave);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const float xa = rs_xor32(acc[2 * m][0], acc[2 * m][2]), ya = rs_xor32(acc[2 * m + 1][0], acc[2 * m + 1][2]);
            const float xb = rs_xor32(acc[2 * m][1], acc[2 * m][3]), yb = rs_xor32(acc[2 * m + 1][1], acc[2 * m + 1][3]);
            dims(xa, ya, z_a, inv_a, o[0][2 * m], o[0][2 * m + 1]);
            dims(xb, yb, z_b, inv_b, o[1][2 * m], o[1][2 * m + 1]);
        }
    }
}

// Rows of one split into image slot j; lanes 0 .. G-1 write the LSE of head n.
template <int G, class Cap, bool V3 = false>
__device__ __forceinline__ void stash_split(const State &st, const floatx4 (&acc)[8], const LaneConst &lc,
                                            float *img, int j) {
    int h0;
    float o[G / 4][8], safe_l;
    finish_rows<G, V3>(st, acc, lc, h0, o, safe_l);
    float *r = img + h0 * Cap::head_floats + j * (kHeadDim + 1) + 8 * lc.n;
#pragma unroll
    for (int k = 0; k < G / 4; ++k)
#pragma unroll
        for (int i = 0; i < 8; ++i)
            r[k * Cap::head_floats + i] = o[k][i];
    if (lc.g == 0 && lc.n < G)
        img[lc.n * Cap::head_floats + j * (kHeadDim + 1) + kHeadDim] = lse_of(st.negm, safe_l);
}

// Output element conversion of the fused epilogue (the same roundings as Stage2's).
__device__ __forceinline__ void put_out(void *out, int dtype, int64_t i, float v) {
    if (dtype == kOutBf16)
        static_cast<__bf16 *>(out)[i] = (__bf16)v;
    else if (dtype == kOutF16)
        static_cast<_Float16 *>(out)[i] = (_Float16)v;
    else
        static_cast<float *>(out)[i] = v;
}

// One split per sequence: with a single live split Stage2's merge is the identity (weight
// exp(0) = 1, sum 1), so the wave writes the final output rows and LSE itself -- the same
// values Stage2 would write, without the mid_o round trip.
// Heads nh .. G-1 of the wave are padding (a GQA group that is not a multiple of G).
template <int G>
__device__ __forceinline__ void emit_output(const State &st, const floatx4 (&acc)[8], const LaneConst &lc,
                                            void *out, int out_dtype, float *lse, int64_t row0, int nh) {
    int h0;
    float o[G / 4][8], safe_l;
    finish_rows<G, false>(st, acc, lc, h0, o, safe_l);
    const int64_t r = (row0 + h0) * kHeadDim + 8 * lc.n;
#pragma unroll
    for (int k = 0; k < G / 4; ++k)
        if (h0 + k < nh)
#pragma unroll
            for (int i = 0; i < 8; ++i)
                put_out(out, out_dtype, r + k * kHeadDim + i, o[k][i]);
    if (lc.g == 0 && lc.n < nh)
        lse[row0 + lc.n] = lse_of(st.negm, safe_l);
}

// Write image slots 0 .. ns-1 to the rows of splits s0 .. s0+ns-1 (heads 0 .. nh-1; the
// rest are padding).  Rows of one head and consecutive splits are consecutive in mid_o
// [B, Hq, S, D + 1], so head h's slots are one run of ns * 129 floats.  One wave: its LDS
// accesses complete in program order, so only the compiler must keep the image reads after
// the writes.
template <int G, class Cap>
__device__ __forceinline__ void flush_splits(const float *img, float *__restrict__ mid_o, int64_t row0,
                                             int num_splits, int s0, int ns, int lane, int nh) {
    asm volatile("" ::: "memory");
    const int64_t head_bytes = (int64_t)num_splits * (kHeadDim + 1) * 4;
    float *base = mid_o + (row0 * num_splits + s0) * (kHeadDim + 1);
    const __amdgpu_buffer_rsrc_t out = __builtin_amdgcn_make_buffer_rsrc(base, 0, 0x7FFFFFFF, 0x00020000);
    const int run = ns * (kHeadDim + 1);  // floats per head
    const int chunks = run >> 2;
#pragma unroll
    for (int h = 0; h < G; ++h) {
        if (h >= nh)
            break;
        const float *src = img + h * Cap::head_floats;
        for (int c = lane; c < chunks; c += kWave) {
            const float4 v = *reinterpret_cast<const float4 *>(src + 4 * c);
            __builtin_amdgcn_raw_buffer_store_b128(
                u32x4{__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)}, out,
                (int)(h * head_bytes) + 16 * c, 0, 0);
        }
        if (lane < (run & 3))
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(src[4 * chunks + lane]), out,
                                                  (int)(h * head_bytes) + 16 * chunks + 4 * lane, 0, 0);
    }
    asm volatile("" ::: "memory");
}

// ---- Query rotation inside the one-split kernel (ROT) --------------------------------
// A workgroup holds the nvh waves of one sequence (nvh = its kv-heads times the parts of
// their GQA groups, a divisor of 8: at most two waves per SIMD of one CU).  Together they
// compute the sequence's rotated queries q_rot = query @ rot_t into LDS with the operands
// and the MFMA order of rotate_mfma_kernel, so the rows are bit-identical to that launch's:
// each query row scaled by the power of two that puts its largest |x| in [2^14, 2^15) (exact
// in f16 for fp16 / bf16 queries), rot_t as f16 hi + lo parts, D[rows 4g .. 4g+3][col n] of
// output column tile c per row tile.  Wave w takes the column tiles c = w, w + nvh, ..., so it
// reads 8 KB of rot_t per tile (one column slab), not the whole 64 KB.
constexpr int kRotGroupWaves = 8;
constexpr int kQRowFloats = kHeadDim + 4;  // LDS row of a rotated query (rows 16 bytes apart in bank)

// Query elements of the lane for every row tile of the sequence: row 16t + n (rows past Hq
// repeat the last one and are not stored), elements 32kb + 8g .. +7 -- the A operand of
// rotate_mfma_kernel.  Hq <= 8 G, so G / 2 row tiles.
template <int G> struct RotRows {
    uint4 raw[G / 2][4];
};
template <typename InT, int G>
__device__ __forceinline__ void rot_load_rows(RotRows<G> &a, const InT *__restrict__ query, int64_t row_base,
                                              int hq, int n, int g) {
#pragma unroll
    for (int t = 0; t < G / 2; ++t) {
        const int row = min(16 * t + n, hq - 1);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
            a.raw[t][kb] = *reinterpret_cast<const uint4 *>(query + (row_base + row) * kHeadDim + 32 * kb + 8 * g);
    }
}
// rot_t[32kb + 8g + j][16c + n]: the lane's B operand of column tile c (fp32, split later).
struct RotCols {
    float v[4][8];
};
__device__ __forceinline__ void rot_load_cols(RotCols &b, const float *__restrict__ rot_t, int c, int n, int g) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j)
            b.v[kb][j] = rot_t[(32 * kb + 8 * g + j) * kHeadDim + 16 * c + n];
}
// Scaled f16 A operands of every row tile and the scale exponents of the D rows each lane
// receives (row 4g + i of tile t).
template <typename InT, int G>
__device__ __forceinline__ void rot_a_operands(const RotRows<G> &a, half8 (&ah)[G / 2][4], int (&e_out)[G / 2][4],
                                               int g) {
    typedef InT in8 __attribute__((ext_vector_type(8)));
#pragma unroll
    for (int t = 0; t < G / 2; ++t) {
        float amax = 0.f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const in8 p = __builtin_bit_cast(in8, a.raw[t][kb]);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                amax = fmaxf(amax, fabsf(to_float<InT>(p[j])));
        }
        amax = rot_row_max(amax);
        const int e = (amax > 0.f && amax < __builtin_inff()) ? 15 - __builtin_amdgcn_frexp_expf(amax) : 0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            e_out[t][i] = __shfl(e, 4 * g + i, kWave);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const in8 p = __builtin_bit_cast(in8, a.raw[t][kb]);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                ah[t][kb][j] = (_Float16)__builtin_ldexpf(to_float<InT>(p[j]), e);
        }
    }
}
// Column tile c of every row tile into the LDS rows qbuf [Hq][kQRowFloats].
template <int G>
__device__ __forceinline__ void rot_column_tile(const half8 (&ah)[G / 2][4], const int (&e_out)[G / 2][4],
                                                const RotCols &b, float *qbuf, int c, int hq, int n, int g) {
    half8 bh[4], bl[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            bh[kb][j] = (_Float16)b.v[kb][j];
            bl[kb][j] = (_Float16)(b.v[kb][j] - (float)bh[kb][j]);
        }
#pragma unroll
    for (int t = 0; t < G / 2; ++t) {
        if (16 * t >= hq)
            break;
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            acc = mfma(ah[t][kb], bh[kb], acc);
            acc = mfma(ah[t][kb], bl[kb], acc);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 16 * t + 4 * g + i;
            if (row < hq)
                qbuf[row * kQRowFloats + 16 * c + n] = __builtin_ldexpf(acc[i], -e_out[t][i]);
        }
    }
}

// One wave handles a run of consecutive live splits of one (sequence, kv-head).  Their
// tiles form one stream: split s contributes its n_s tiles padded to an even count, the
// wave's last split as many more as make the stream whole ring turns (padding positions
// re-read the split's last tile and mask every token), so split ends fall after an odd
// stage, with the PV of the split's last pair of positions.  After a split's last
// stage the wave puts its rows into the LDS image (flushed to mid_o when full and after
// the wave's last split) and restarts the softmax state and the accumulators.
//
// GQA groups: a wave serves G (4 or 8) q-heads of one kv-head.  A group of more than G
// heads is served by parts of G heads (ceil(group / G) waves per kv-head, each reading the
// kv-head's tiles), and a group that is not a multiple of G leaves the last part's heads
// nh .. G-1 as padding (zero queries, never written).  Grid x runs over the (part, kv-head)
// pairs, vh = part * Hk + kv-head.
//
// FUSED (launched with one split per sequence and one wave per (sequence, kv-head part)): the
// wave writes the final output rows (out, out_dtype) and LSE instead of mid_o rows.
// ROT (with FUSED; 1: bf16 queries, 2: fp16): a workgroup is the nvh waves of one sequence
// (grid (B)), which rotate the query themselves (q_rot is not read: `query`, `rot_t`, and
// pair_lut holds the 16 centroids).
// KF8: the FP8-key preset (K one E4M3 byte per dim, no norm, the query not rotated).
// KB3: the 3-bit-key / 4-bit-value preset (pair_lut then holds the 8 centroids).
template <int LAYOUT, int G, int WPE, bool FUSED, bool KF8 = false, bool KB3 = false, bool V3 = false, int ROT = 0>
__global__ __launch_bounds__(ROT ? kWave * kRotGroupWaves : kWave) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void stage1_xdl_kernel(
    const float *__restrict__ q_rot, const uint8_t *__restrict__ cache,
    const int32_t *__restrict__ block_table, const int32_t *__restrict__ seq_lens,
    const float *__restrict__ pair_lut, float *__restrict__ mid_o, const float *__restrict__ sinks,
    void *__restrict__ out, int out_dtype, float *__restrict__ lse,
    int num_q_heads, int num_kv_heads, int block_size_log2, int max_blocks, int64_t block_stride,
    int slot_pos, int slot_head, int num_splits, float score_scale_log2,
    const void *__restrict__ query, const float *__restrict__ rot_t) {
    static_assert(G == 4 || G == 8, "4 or 8 q-heads per wave");
    static_assert(ROT == 0 || (FUSED && !KF8 && !KB3), "the query rotation runs in the one-split 4-bit kernel");
    using QueryT = std::conditional_t<ROT == 1, __bf16, _Float16>;
    constexpr int TPL = G / 4;
    constexpr int RING = 4;
    // ring slots of the first chunk issued before the K table and q operands are built (the
    // rest after): with every wave of the launch asking at once, a wave's first tiles then
    // queue behind fewer of the other waves' loads
    constexpr int FIRST_SLOTS = 2;
    const int block_size = 1 << block_size_log2;
    int vh, wid, b;
    if constexpr (ROT) {
        // wave w of the sequence's workgroup; with 8 waves (2 per SIMD: waves w and w + 4 share
        // one) SIMD s gets parts 2s and 2s + 1, one even and one odd kv-head (see below)
        const int w = threadIdx.x / kWave;
        vh = blockDim.x == kWave * 8 ? 2 * (w & 3) + (w >> 2) : w;
        wid = 0;
        b = blockIdx.x;
    } else {
        vh = blockIdx.x;
        wid = blockIdx.y;
        b = blockIdx.z;
    }
    const int nw = ROT ? 1 : gridDim.y;
    if constexpr (!ROT && (LAYOUT == 1 || KF8 || KB3)) {
        // Workgroups are dealt to the XCDs round-robin by linear id (8 on gfx950), so with
        // the plain map kv-head h runs on XCD h.  An AoS slot (or a preset's SoA record of
        // 192, 112 or 96 bytes) of kv-head h shares 128-byte lines with those of h - 1 and h + 1: the kv-heads of one (sequence, wave)
        // pair go to one XCD instead, so each line is fetched from HBM into one L2 (halves
        // the HBM reads).  A bijection of the grid whenever the pair count is a multiple of 8.
        constexpr int kXcds = 8;
        const int hk = gridDim.x, pairs = gridDim.y * gridDim.z;
        if (pairs % kXcds == 0) {
            const int lin = blockIdx.x + hk * (blockIdx.y + gridDim.y * blockIdx.z);
            const int r = lin / kXcds;
            const int pair = lin % kXcds + kXcds * (r / hk);
            vh = r % hk;
            wid = pair % nw;
            b = pair / nw;
        }
    }
    // The two waves of a SIMD are workgroups i and i + half the grid (one round at 2 waves
    // per SIMD), and with either map above both would serve the same kv-head.  kv-heads read
    // HBM at different speeds by where their records sit in the cache rows (4-bit SoA: the
    // odd ones, upper halves of 256-byte stretches, ~7 % slower), so SIMDs holding two slow
    // ones would end last: the second half of the grid takes kv-head h ^ 1 instead, and
    // every SIMD runs one even and one odd kv-head.  The kv-heads of one (sequence, wave)
    // pair still start together (and share an XCD where the map above puts them on one).
    if (!ROT && (gridDim.x & 1) == 0 && 2 * (wid + nw * b) >= nw * (int)gridDim.z)
        vh ^= 1;
    const int lane = threadIdx.x % kWave;
    const int group = num_q_heads / num_kv_heads;
    const int kvh = vh % num_kv_heads, part = vh / num_kv_heads;
    const int hb = kvh * group + part * G;       // the wave's first q-head
    const int nh = min(G, group - part * G);     // its real q-heads (the rest are padding)
    const int hl = min((lane & 15) & (G - 1), nh - 1);  // the lane's q-head (padding: a real one's)
    // Block-table entries of the wave's first tiles, loaded while seq_lens and the wave deal
    // are worked out: a guess (the grid's own sequence and run at full length) that equal
    // lengths make right.  When the first chunk's entries turn out to be exactly these, the
    // registers serve it and the block-table read leaves the path to the first KV loads;
    // otherwise the guess has warmed L2 for the real reads.
    const int guess_b = b, guess_first = wid * ((max_blocks + nw - 1) / nw);
    const int bt_guess = block_table[(int64_t)b * max_blocks + min(guess_first + lane, max_blocks - 1)];
    // The pair-LUT rows do not depend on the sequence: they go out first; the K table and the
    // q operands are built once the first tiles' loads are on their way.
    static_assert(!(KF8 && KB3), "one key format");
    static_assert(!V3 || (KB3 && !FUSED), "3-bit values come with 3-bit keys, not fused");
    // 3-bit presets, SoA: records staged through LDS (RawRec), see stage_records
    constexpr bool STG = KB3 && LAYOUT == 0;
    // FP8 keys, SoA: records staged the same way (RawRec3)
    constexpr bool STG8 = KF8 && LAYOUT == 0;
    using RK = std::conditional_t<STG8, RawRec3, std::conditional_t<KF8, RawK8, std::conditional_t<STG, RawRec, std::conditional_t<KB3, RawK3, RawK<LAYOUT>>>>>;
    LutRows lut_rows{};
    if constexpr (ROT) {
        // from the centroids themselves: entry e = (c[e & 15], c[e >> 4]), the pair-LUT row
#pragma unroll
        for (int i = 0; i < 256 / kWave; ++i) {
            const int e = lane + kWave * i;
            lut_rows.r[i] = float2{pair_lut[e & 15], pair_lut[e >> 4]};
        }
    } else if constexpr (!KF8 && !KB3) {
        lut_rows = load_lut_rows(pair_lut, lane);
    }
    // the head's sink logit (a dummy read when there are none: one unconditional load here
    // keeps the waits before the first KV loads from covering it)
    const float sink = *(sinks ? sinks + hb + hl : q_rot);
    int run_waves = nw;  // waves sharing this wave's sequence and kv-head
    int dealt_len = 0;
    if constexpr (!FUSED) {
        const Deal d = deal_waves(seq_lens, gridDim.z, num_splits, nw, wid + nw * b, lane);
        if (d.b < 0)
            return;
        b = d.b;
        wid = d.wid;
        run_waves = d.nw;
        dealt_len = d.len;
    }
    const int seq_len = FUSED ? seq_lens[b] : dealt_len;
    // split partition: L = ceil(len / S); live splits are those with s * L < len
    const int split_len = div_pos(max(seq_len, 0) + num_splits - 1, num_splits);
    const int live = split_len > 0 ? min(num_splits, div_pos(seq_len + split_len - 1, split_len)) : 0;
    // run x of the W runs of this (sequence, kv-head): live splits from x q + min(x, r), q + 1 of
    // them for x < r and q after (q = live / W, r = live % W)
    const int run_q = div_pos(live, run_waves), run_r = live - run_q * run_waves;
    const int s_lo = wid * run_q + min(wid, run_r);
    const int s_hi = s_lo + run_q + (wid < run_r ? 1 : 0);
    if constexpr (FUSED) {
        if (live == 0) {
            // an empty sequence: what Stage2 writes for it (0 / 0 and ln 0); with ROT every
            // wave of the workgroup returns here (one sequence), before its barrier
            const int64_t r0 = ((int64_t)b * num_q_heads + hb) * kHeadDim;
            for (int i = lane; i < nh * kHeadDim; i += kWave)
                put_out(out, out_dtype, r0 + i, __builtin_nanf(""));
            if (lane < nh)
                lse[(int64_t)b * num_q_heads + hb + lane] = -__builtin_inff();
            return;
        }
    }
    if (s_lo >= s_hi)
        return;

    LaneConst lc;
    lc.n = lane & 15;
    lc.g = lane >> 4;
    lc.tok_bit0 = (lc.n >> 2) & 1;
    lc.tok_bit1 = (lc.n >> 3) & 1;
    lc.upper = lc.n >= 8;
    lc.part_sel = lc.upper ? 0x07060302u : 0x05040100u;

    __shared__ uint32_t ktab[KTable<LAYOUT>::words];
    // the stage buffer of the records (3-bit: + 16 bytes, a 3-bit V dword of token 15, n = 15,
    // reads 4 bytes past them and masks them off); the image takes what the K table (none
    // for FP8 keys) and the stage buffer leave
    constexpr int kRec = record_bytes<LAYOUT, KF8, KB3, V3>();
    constexpr int kStage = STG ? 16 * kRec + 16 : STG8 ? 16 * kRec : 0;
    __shared__ __align__(16) uint8_t recbuf[kStage > 0 ? kStage : 16];
    // split starts of a chunk, one byte per stream position (chunk_tiles; one split per wave
    // when FUSED)
    __shared__ uint8_t marks[FUSED ? 1 : kWave];
    using Cap = SpanCap<LAYOUT, G, WPE, (KF8 ? 0 : KTable<LAYOUT>::words * 4) + kStage + (FUSED ? 0 : kWave)>;
    __shared__ __align__(16) float img[FUSED ? 4 : Cap::floats];  // FUSED writes no mid_o rows
    __shared__ __align__(16) float qbuf[ROT ? kRotGroupWaves * G * kQRowFloats : 4];
    half8 bq[8];
    float q_unscale = 1.f;  // 2^-e of the lane's q row (q_operands)

    State st{__FLT_MAX__, 0.f, 0.f, 1.f};
    if (sinks && s_lo == 0) {
        // split 0 starts from the head's sink logit: max = sink, sum = 1 (one lane per head,
        // lane h, holds it; the sums are totalled over the lanes n = h (mod G))
        st.negm = -sink * kLog2e;
        st.l = lane < G ? 1.f : 0.f;
    }
    floatx4 acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
        acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // Stream positions of split s: its tiles rounded up to an even count (a split ends
    // after an odd stage, with the PV of its last pair); the wave's last split takes the
    // extra positions that make the stream a whole number of ring turns.
    auto split_tiles = [&](int s) {
        const int st0 = s * split_len, en = min(st0 + split_len, seq_len);
        return ((en - 1) >> 4) - (st0 >> 4) + 1;
    };
    // A run of at most 64 splits keeps them in lanes (lane i: split s_lo + i): first tile,
    // tile count and the stream position where the split starts.  Lane-parallel, this takes a
    // few instructions where loops over the splits took hundreds (all of a CU's waves run
    // their prologue at once).
    const int n_run = s_hi - s_lo;
    const bool run_in_lanes = n_run <= kWave;
    int sp_tf = 0, sp_nt = 0, sp_base = 0;
    int e_log2 = -1;  // log2 of the positions of every split of the run when they are one power of two
    int total = 0;
    if (run_in_lanes) {
        const int st0 = (s_lo + min(lane, n_run - 1)) * split_len, en = min(st0 + split_len, seq_len);
        sp_tf = st0 >> 4;
        sp_nt = ((en - 1) >> 4) - sp_tf + 1;
        const int e = lane < n_run ? (sp_nt + 1) & ~1 : 0;
        const int incl = (int)wave_scan((uint32_t)e);
        sp_base = incl - e;
        total = __builtin_amdgcn_readlane(incl, kWave - 1);
        const int e0 = __builtin_amdgcn_readfirstlane(e);
        if (__ballot(lane < n_run && e != e0) == 0 && (e0 & (e0 - 1)) == 0)
            e_log2 = __builtin_ctz((unsigned)e0);
    } else {
        for (int s = s_lo; s < s_hi; ++s)
            total += (split_tiles(s) + 1) & ~1;
    }
    const int tail = ((total + RING - 1) & ~(RING - 1)) - total;
    total += tail;
    auto split_stop = [&](int s) { return ((split_tiles(s) + 1) & ~1) + (s == s_hi - 1 ? tail : 0); };

    const LaneOffsets off =
        lane_offsets<LAYOUT, G, KF8, KB3, V3>(lc.n, lc.g, kvh, num_kv_heads, block_size, slot_pos, slot_head);
    const int32_t *bt = block_table + (int64_t)b * max_blocks;
    const int tok0 = 4 * lc.g + TPL * (lc.n / G);  // the lane's first softmax token
    const int64_t row0 = (int64_t)b * num_q_heads + hb;
    const int rec = record_bytes<LAYOUT, KF8, KB3, V3>();

    int cur = s_lo;
    int img_s0 = s_lo;  // split of image slot 0
    int cur_start = cur * split_len;
    int cur_end = min(cur_start + split_len, seq_len);
    int cur_stop = split_stop(cur);

    // Lane i of base_lo / base_hi holds the address of the 16-token piece at stream
    // position j0 + i of the current chunk (its KV block plus the piece's offset), lane i
    // of moff_lane the SoA metadata offset relative to that address.
    auto rsrc_at = [&](uint32_t base_lo, uint32_t base_hi, int j) {
        const uint64_t a = ((uint64_t)__builtin_amdgcn_readlane(base_hi, j & 63) << 32) |
                           (uint32_t)__builtin_amdgcn_readlane(base_lo, j & 63);
        return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void *>(a), 0, 0x7FFFFFFF, 0x00020000);
    };
    // The scheduling barriers keep the loads in program order, which is what lets each
    // wait count only the loads of later tiles.
    // A position's descriptor is built for its K load and kept for its V load, issued one or
    // two stages later: pos[p & 3] holds position p's (positions j + 4 .. j + 8 around
    // stage j, and j is a multiple of 4).
    auto issue_kpos = [&](RK &r, const __amdgpu_buffer_rsrc_t &rsrc) {
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (KF8 || KB3)
            issue_k(r, rsrc, 0, off);
        else
            issue_k<LAYOUT>(r, rsrc, 0, off);
        __builtin_amdgcn_sched_barrier(0);
    };
    auto issue_vpos = [&](RawV<LAYOUT, TPL> &r, const __amdgpu_buffer_rsrc_t &rsrc, int moff_lane, int j) {
        const int moff = LAYOUT == 0 ? __builtin_amdgcn_readlane(moff_lane, j & 63) : 0;
        __builtin_amdgcn_sched_barrier(0);
        issue_v<LAYOUT, TPL, KF8, KB3, V3>(r, rsrc, 0, moff, off);
        __builtin_amdgcn_sched_barrier(0);
    };

    floatx4 sc;         // QK^T accumulator of the next tile
    std::conditional_t<KF8, K8, std::conditional_t<KB3, RawK3, uint4>> kn;  // K bytes of the next tile, in the MFMA layout
    float csq_tot = 0;  // AoS: ||c[idx]||^2 of token n of that tile
    uint32_t aw[4];

    // Stage j: softmax of position j, then QK^T of position j + 1; odd stages also run
    // the PV of positions (j - 1, j).
    auto stage = [&](int k, const RawV<LAYOUT, TPL> &vprev, const RawV<LAYOUT, TPL> &vcur,
                     const RK &kafter, RawV<LAYOUT, TPL> &vafter, int mask_lane, int j) {
        // K-table lookups of the next tile first: their latency runs under the softmax
        KOps e;
        if constexpr (KF8)
            e = lookup_tile(kn, ktab);
        else
            e = lookup_tile<LAYOUT>(kn, ktab);
        __builtin_amdgcn_sched_barrier(0);
        const TileV t = decode_v<LAYOUT, TPL>(vcur, off);
        const int t0 = 16 * __builtin_amdgcn_readlane(mask_lane, j & 63);
        const bool boundary = !(t0 >= cur_start && t0 + 16 <= cur_end);
        float dot[TPL], nf[TPL];
        bool valid[TPL];
        lane_dots<G>(sc, lc, dot);
#pragma unroll
        for (int q = 0; q < TPL; ++q) {
            valid[q] = (uint32_t)(t0 + tok0 + q - cur_start) < (uint32_t)(cur_end - cur_start);
            if constexpr (LAYOUT == 0 || KF8) {
                nf[q] = half_at(t.norm, q) * q_unscale;
            } else {
                // ||c[idx]||^2 of token tok0 + q: totals sit in lanes n = token (any row)
                nf[q] = half_at(t.norm, q) * __builtin_amdgcn_rsqf(__shfl(csq_tot, tok0 + q, kWave) + 1e-16f) *
                        q_unscale;
            }
        }
        if (k & 1)
            softmax_tile<G, true>(dot, nf, t, st, acc, lc, boundary, valid, aw[0], aw[1], aw[2], aw[3]);
        else
            softmax_tile<G, false>(dot, nf, t, st, acc, lc, boundary, valid, aw[0], aw[1], aw[0], aw[1]);
        if (k & 1) {
            const TileV ta = decode_v<LAYOUT, TPL>(vprev, off);
            sc = pv_qk<V3>(acc, aw, ta.v, t.v, e, bq);
        } else {
            sc = qk_tile(e, bq);
        }
        if constexpr (LAYOUT == 1 && !KF8)
            csq_tot = sum_xor16(sum_xor32(e.csq));
        // K bytes of position j + 2 into the MFMA layout (its load was issued 3 stages ago);
        // staged records also give its V codes
        if constexpr (STG)
            kn = stage_records<kRec, V3>(kafter, recbuf, off, vafter.v);
        else if constexpr (STG8)
            kn = stage_records(kafter, recbuf, off, vafter.v);
        else if constexpr (KF8 || KB3)
            kn = decode_k(kafter, off);
        else
            kn = decode_k<LAYOUT>(kafter, off);
    };

    // Stream positions in chunks of 64 (one block-table entry per lane).  K loads of
    // position j + 5 are issued right after QK^T of j + 1 consumed its slot; V loads of
    // positions j + 3, j + 4 after the PV of (j - 1, j).  Every load and stage is
    // unconditional -- past the chunk's end a load re-reads its last tile (an L2 hit) --
    // so all paths issue the same loads in the same order.
    // chunk state: lane i holds stream position j0 + i's tile, mask and address
    int tile_lane = 0, mask_lane = 0, moff_lane = 0;
    uint32_t base_lo = 0, base_hi = 0;
    RK kr[RING];
    RawV<LAYOUT, TPL> vr[RING];
    __amdgpu_buffer_rsrc_t pos[RING];
    // Lane tables of chunk [j0, j0 + 64) and the ring's first loads.
    // ring slots k0 .. k1-1 of the chunk at j0: K and V loads of positions j0 + k
    auto issue_slots = [&](int j0, int last, int k0, int k1) {
#pragma unroll
        for (int k = 0; k < RING; ++k) {
            if (k < k0 || k >= k1)
                continue;
            const auto rsrc = rsrc_at(base_lo, base_hi, min(j0 + k, last));
            issue_kpos(kr[k], rsrc);
            issue_vpos(vr[k], rsrc, moff_lane, min(j0 + k, last));
        }
    };
    // Lane i: the tile and mask of stream position j0 + i and the block-table entry of that
    // tile (read here; the addresses come from chunk_addresses).
    auto chunk_tiles = [&](int j0, int nchunk) {
        if (run_in_lanes && e_log2 >= 0) {
            // every split takes 2^e_log2 positions (the tail's go to the last one)
            const int p = j0 + min(lane, nchunk - 1);
            const int i = min(p >> e_log2, n_run - 1);
            const int st0 = (s_lo + i) * split_len, en = min(st0 + split_len, seq_len);
            const int tf = st0 >> 4, nt = ((en - 1) >> 4) - tf + 1, o = p - (i << e_log2);
            tile_lane = tf + min(o, nt - 1);
            mask_lane = o < nt ? tile_lane : -(1 << 24);  // padding: no valid token
        } else if (run_in_lanes) {
            int i = 0;  // the lane's split, as an index into the run
            if constexpr (!FUSED) {
                if (n_run > 1) {
                    // the splits that start inside (j0, j0 + 64) mark their offset; position
                    // j0 + q lies in the split that holds j0, moved on by the marks up to q
                    marks[lane] = 0;
                    const int q = sp_base - j0;
                    if (lane < n_run && q > 0 && q < kWave)
                        marks[q] = 1;
                    // other lanes' marks: the compiler must not forward the lane's own stores
                    // (one wave: its LDS writes complete before its later reads)
                    asm volatile("" ::: "memory");
                    const uint64_t m = __ballot(marks[lane] != 0);
                    const int i0 = __builtin_popcountll(__ballot(lane < n_run && sp_base <= j0)) - 1;
                    i = __shfl(i0 + __builtin_popcountll(m & (~0ull >> (63 - lane))), min(lane, nchunk - 1), kWave);
                }
            }
            const int o = j0 + min(lane, nchunk - 1) - __shfl(sp_base, i, kWave);
            const int nt = __shfl(sp_nt, i, kWave);
            tile_lane = __shfl(sp_tf, i, kWave) + min(o, nt - 1);
            mask_lane = o < nt ? tile_lane : -(1 << 24);  // padding: no valid token
        } else {
            const int p = j0 + min(lane, nchunk - 1);
            int base = 0;
            tile_lane = 0;
            mask_lane = 0;
            for (int s = s_lo; s < s_hi; ++s) {
                const int st0 = s * split_len, en = min(st0 + split_len, seq_len);
                const int tf = st0 >> 4, nt = ((en - 1) >> 4) - tf + 1;
                if (p >= base) {
                    const int o = p - base;
                    tile_lane = tf + min(o, nt - 1);
                    mask_lane = o < nt ? tile_lane : -(1 << 24);  // padding: no valid token
                }
                base += split_stop(s);
            }
        }
        const int bidx = (16 * tile_lane) >> block_size_log2;
        const bool guessed = j0 == 0 && b == guess_b &&
                             __ballot(bidx != min(guess_first + lane, max_blocks - 1)) == 0;
        return guessed ? bt_guess : bt[bidx];
    };
    auto chunk_addresses = [&](int blk) {
        {
            const int toff = (16 * tile_lane) & (block_size - 1);
            // the piece's first record: token toff of kv-head 0 (AoS: at toff * slot_pos)
            const int piece = LAYOUT == 0 ? toff * num_kv_heads * rec : toff * slot_pos;
            const uint64_t a = reinterpret_cast<uint64_t>(cache) + (uint64_t)((int64_t)blk * block_stride) +
                               (uint64_t)piece;
            base_lo = (uint32_t)a;
            base_hi = (uint32_t)(a >> 32);
            moff_lane = (block_size - toff) * num_kv_heads * rec + toff * 2;
        }
    };
    auto open_chunk = [&](int j0, int nchunk, int last, int nslots) {
        chunk_addresses(chunk_tiles(j0, nchunk));
        issue_slots(j0, last, 0, nslots);
    };

    // The first chunk's first loads go out before the K table and the q operands are built,
    // and the q (or rotation) loads between its block-table read and those: loads complete in
    // issue order, so the first KV addresses wait for the block table alone and the q rows
    // arrive under the first KV loads.
    const int blk0 = chunk_tiles(0, min(64, total));
    float4 q_rows[8];
    RotRows<G> rot_rows;
    RotCols rot_cols;
    const int nvh = ROT ? (int)(blockDim.x / kWave) : 1;
    if constexpr (ROT) {
        rot_load_rows<QueryT, G>(rot_rows, static_cast<const QueryT *>(query), (int64_t)b * num_q_heads,
                                 num_q_heads, lane & 15, lane >> 4);
        rot_load_cols(rot_cols, rot_t, threadIdx.x / kWave, lane & 15, lane >> 4);
    } else {
        load_q_rows(q_rows, q_rot, (int64_t)b * num_q_heads + hb + hl, lane >> 4, KF8);
    }
    chunk_addresses(blk0);
    issue_slots(0, min(64, total) - 1, 0, FIRST_SLOTS);
    if constexpr (ROT) {
        // the sequence's rotated queries into qbuf (column tiles w, w + nvh, ... of this wave)
        half8 ah[G / 2][4];
        int e_out[G / 2][4];
        rot_a_operands<QueryT, G>(rot_rows, ah, e_out, lc.g);
        const int w = threadIdx.x / kWave;
        rot_column_tile<G>(ah, e_out, rot_cols, qbuf, w, num_q_heads, lc.n, lc.g);
        for (int c = w + nvh; c < kHeadDim / 16; c += nvh) {
            rot_load_cols(rot_cols, rot_t, c, lc.n, lc.g);
            rot_column_tile<G>(ah, e_out, rot_cols, qbuf, c, num_q_heads, lc.n, lc.g);
        }
        // the shared K table: wave w builds rows i = w (mod nvh) of it
        build_key_table_rows<LAYOUT>(ktab, lut_rows, lane, w, nvh);
        // LDS writes done, then the workgroup barrier (the KV loads stay in flight: no
        // vmcnt wait, unlike __syncthreads)
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
        for (int m = 0; m < 8; ++m)
            q_rows[m] = *reinterpret_cast<const float4 *>(qbuf + (hb + hl) * kQRowFloats + 32 * lc.g + 4 * m);
        if (hl != ((lane & 15) & (G - 1)))
#pragma unroll
            for (int m = 0; m < 8; ++m)
                q_rows[m] = float4{0.f, 0.f, 0.f, 0.f};
    } else {
        if (hl != ((lane & 15) & (G - 1)))  // padding head: a zero query
#pragma unroll
            for (int m = 0; m < 8; ++m)
                q_rows[m] = float4{0.f, 0.f, 0.f, 0.f};
        if constexpr (KB3)
            build_key_table3(ktab, pair_lut, lane);
        else if constexpr (!KF8)
            build_key_table<LAYOUT>(ktab, lut_rows, lane);
    }
    q_unscale = q_operands(bq, q_rows, lc.n, score_scale_log2);
    issue_slots(0, min(64, total) - 1, FIRST_SLOTS, RING);
    // one wave: its LDS writes complete before its later LDS reads; only the compiler must
    // keep the table lookups after the build
    asm volatile("" ::: "memory");

    int pos_base = 0;  // stream position where split `cur` starts
    for (int j0 = 0; j0 < total; j0 += 64) {
        const int nchunk = min(64, total - j0);
        const int last = j0 + nchunk - 1;
        if (j0 > 0)
            open_chunk(j0, nchunk, last, RING);
        if constexpr (STG8) {
            sc = qk_tile(lookup_tile(stage_records(kr[0], recbuf, off, vr[0].v), ktab), bq);
            kn = stage_records(kr[1], recbuf, off, vr[1].v);
        } else if constexpr (KF8) {
            sc = qk_tile(lookup_tile(decode_k(kr[0], off), ktab), bq);
            kn = decode_k(kr[1], off);
        } else if constexpr (STG) {
            sc = qk_tile(lookup_tile<LAYOUT>(stage_records<kRec, V3>(kr[0], recbuf, off, vr[0].v), ktab), bq);
            kn = stage_records<kRec, V3>(kr[1], recbuf, off, vr[1].v);
        } else if constexpr (KB3) {
            const KOps e = lookup_tile<LAYOUT>(decode_k(kr[0], off), ktab);
            sc = qk_tile(e, bq);
            if constexpr (LAYOUT == 1)
                csq_tot = sum_xor16(sum_xor32(e.csq));
            kn = decode_k(kr[1], off);
        } else {
            const KOps e = lookup_tile<LAYOUT>(decode_k<LAYOUT>(kr[0], off), ktab);
            sc = qk_tile(e, bq);
            if constexpr (LAYOUT == 1)
                csq_tot = sum_xor16(sum_xor32(e.csq));
            kn = decode_k<LAYOUT>(kr[1], off);
        }
        pos[0] = rsrc_at(base_lo, base_hi, min(j0 + RING, last));
        issue_kpos(kr[0], pos[0]);
        int j = j0;
        do {
#pragma unroll
            for (int k = 0; k < RING; ++k) {
                stage(k, vr[(k + RING - 1) % RING], vr[k], kr[(k + 2) % RING], vr[(k + 2) % RING], mask_lane, j + k);
                pos[(k + 1) % RING] = rsrc_at(base_lo, base_hi, min(j + k + 1 + RING, last));
                issue_kpos(kr[(k + 1) % RING], pos[(k + 1) % RING]);
                if (k & 1) {
                    issue_vpos(vr[k - 1], pos[(k + 3) % RING], moff_lane, min(j + k - 1 + RING, last));
                    issue_vpos(vr[k], pos[k % RING], moff_lane, min(j + k + RING, last));
                    // a split ends after an odd stage (FUSED: the only split ends with the
                    // stream; its rows are written after the loop)
                    if (!FUSED && j + k + 1 == pos_base + cur_stop) {
                        stash_split<G, Cap, V3>(st, acc, lc, img, cur - img_s0);
                        if (cur + 1 == s_hi || cur + 1 - img_s0 == Cap::splits) {
                            flush_splits<G, Cap>(img, mid_o, row0, num_splits, img_s0, cur + 1 - img_s0, lane, nh);
                            img_s0 = cur + 1;
                        }
                        // fresh softmax state; the next split's first max change owes nothing
                        st = State{__FLT_MAX__, 0.f, 0.f, 1.f};
#pragma unroll
                        for (int i = 0; i < 8; ++i)
                            acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
                        pos_base = j + k + 1;
                        ++cur;
                        cur_start = cur * split_len;
                        cur_end = min(cur_start + split_len, seq_len);
                        cur_stop = split_stop(cur);
                    }
                }
            }
            j += RING;
        } while (j <= last);
    }
    if constexpr (FUSED)
        emit_output<G>(st, acc, lc, out, out_dtype, lse, row0, nh);
}

}  // namespace xdl
}  // namespace tq4
