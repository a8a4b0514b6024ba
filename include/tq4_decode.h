/*
 * tq4_decode.h -- C ABI of the MI355X (gfx950) TurboQuant `turboquant_4bit_nc`
 * decode path: Stage1 split-KV attention over the 4-bit paged cache, the Stage2
 * split reduction, and the query-rotation / pair-LUT prologue of a full step; the
 * cache writers; and the other presets' Stage1 and writers (FP8 keys
 * `turboquant_k8v4`, 3-bit keys `turboquant_k3v4_nc` / `turboquant_3bit_nc`).
 *
 * All pointers are device pointers; all calls are asynchronous on `stream` and
 * allocate nothing.  Every entry point returns 0 on success, otherwise a
 * nonzero code (TQ4_E_*, or the HIP error of a failed launch) and records a
 * message readable with tq4_last_error() on the calling thread.  Nothing throws.
 *
 * Shapes (row-major, contiguous):
 *   q_rot       float32 [B, Hq, D]            (D == 128; B = batch, 1 .. 65535)
 *   kv_cache    uint8   [num_blocks, block_size, Hk, slot]  slot = 134 at D=128,
 *               physical block stride = cache_block_stride bytes.  Inside a block, SoA
 *               has its own layout; an AoS slot (t, h) starts at (t*Hk + h)*slot
 *               (TQ4_LAYOUT_AOS, position-major) or at (h*block_size + t)*slot
 *               (TQ4_LAYOUT_AOS_HEAD_MAJOR: the vLLM backend's [blocks, Hk, block_size,
 *               slot] cache, which it passes as kv_cache.transpose(1, 2),
 *               reference/turboquant_attn.py:536, :565; the reference AoS kernels take
 *               that view's stride(1) / stride(2), reference/aos_decode.py:563-565,
 *               reference/aos_store.py:375-377)
 *   block_table int32   [B, max_blocks_per_seq]
 *   seq_lens    int32   [B]
 *   pair_lut    float32 [256, 2]              row lo*16+hi = (c[lo], c[hi])
 *   mid_o       float32 [B, Hq, S, D + 1]     S = num_kv_splits (1 .. 65536); [.., D] holds LSE
 *   out         [B, Hq, D] in out_dtype; lse float32 [B, Hq]
 */
#ifndef TQ4_DECODE_H
#define TQ4_DECODE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *tq4_stream_t; /* same type as hipStream_t */

enum tq4_layout { TQ4_LAYOUT_SOA = 0, TQ4_LAYOUT_AOS = 1, TQ4_LAYOUT_AOS_HEAD_MAJOR = 2 };
enum tq4_dtype { TQ4_F32 = 0, TQ4_BF16 = 1, TQ4_F16 = 2 };
enum tq4_kernel {
    TQ4_KERNEL_AUTO = 0,
    TQ4_KERNEL_SIMPLE = 1,
    TQ4_KERNEL_MFMA = 2,   /* retired 4x4x4 MFMA kernel: rejected with TQ4_E_UNSUPPORTED */
    TQ4_KERNEL_XDL = 3
};
enum tq4_status {
    TQ4_OK = 0,
    TQ4_E_INVALID = 1,     /* a shape, pointer or alignment argument is invalid   */
    TQ4_E_UNSUPPORTED = 2  /* valid, but outside the shapes these kernels cover   */
};

/*
 * Stage1: per (sequence b, kv-head, split) partial attention.  Split s covers
 * tokens [s*L, min((s+1)*L, seq_lens[b])) with L = ceil(seq_lens[b] / S); an
 * empty split leaves its mid_o rows untouched.  mid_o[b,h,s,:D] = sum p v / sum p,
 * mid_o[b,h,s,D] = natural-log LSE of the split's scores
 *   score_t = attn_scale * n_t * sum_d q[d] * c[idx_td]
 * (SoA: n_t is the stored folded norm; AoS: raw norm / ||c[idx_t]||).
 * Replaces: launch_tq4_v2_stage1  baseline/triton_v2.py:569-706 (SoA),
 *           launch_soa_v1_stage1  baseline/triton_v1.py:145-203 (SoA),
 *           launch_aos_v1_stage1  baseline/triton_v1.py:90-142  (AoS),
 *           tq4_cuda_vN           cuda/tq4_cuda_v9.cu:276-306, cuda/tq4_cuda_v9_bind.cpp:3-8.
 * The grid depends only on the shapes, never on seq_lens values.
 */
int tq4_stage1(const float *q_rot, const uint8_t *kv_cache, const int32_t *block_table,
               const int32_t *seq_lens, const float *pair_lut, float *mid_o, int B, int Hq,
               int Hk, int D, int block_size, int max_blocks_per_seq,
               int64_t cache_block_stride, int num_kv_splits, int layout, float attn_scale,
               tq4_stream_t stream);

/* Same as tq4_stage1 with an explicit kernel choice (TQ4_KERNEL_*): SIMPLE is the
 * plain-VALU kernel (GQA group 1, 2, 4, 6, 8 or 16); XDL (v_mfma_f32_16x16x32_f16) is the
 * matrix-core kernel (any GQA group: waves of 4 q-heads for groups up to 4, else parts of
 * 8 q-heads, padding heads where the group does not fill them; block_size a power of two
 * >= 16, cache_block_stride a multiple of 16).  AUTO picks XDL when it applies, SIMPLE
 * otherwise.  sinks (fp32 [Hq], may be NULL): per-head sink logits in the score domain
 * (q.k * attn_scale); split 0 starts its softmax with max = sink, sum = 1.
 * Replaces: the per-version entry points tq4_cuda_v1 .. tq4_cuda_v9 (cuda/tq4_cuda_vN_bind.cpp);
 *           the sinks of _tq_decode_stage1 reference/soa_decode_v1.py:134-148. */
int tq4_stage1_ex(const float *q_rot, const uint8_t *kv_cache, const int32_t *block_table,
                  const int32_t *seq_lens, const float *pair_lut, float *mid_o, int B, int Hq,
                  int Hk, int D, int block_size, int max_blocks_per_seq,
                  int64_t cache_block_stride, int num_kv_splits, int layout, float attn_scale,
                  int kernel, const float *sinks, tq4_stream_t stream);

/*
 * Stage2: merge the non-empty splits of every (b, h):
 *   M = max lse_s, w_s = exp(lse_s - M), out = sum w_s o_s / sum w_s, lse = M + ln sum w_s.
 * Replaces: launch_stage2 baseline/stage2.py:58-81 (kernel :8-55);
 *           tq4_cuda_v7_stage2 cuda/tq4_cuda_v7.cu:56-76 (which merges all splits).
 */
int tq4_stage2(const float *mid_o, const int32_t *seq_lens, void *out, int out_dtype,
               float *lse, int B, int Hq, int D, int num_kv_splits, tq4_stream_t stream);

/*
 * q_rot[r, :] = float(query[r, :]) @ rot_t  for r < rows (query in query_dtype).
 * Replaces: `q_rot = (query.float() @ PiT)` reference/soa_decode_v1.py:532-538.
 */
int tq4_rotate_query(const void *query, int query_dtype, const float *rot_t, float *q_rot,
                     int rows, int D, tq4_stream_t stream);

/* pair_lut[lo*n + hi] = (c[lo], c[hi]).  Replaces: build_pair_lut baseline/common.py:232-257. */
int tq4_build_pair_lut(const float *centroids, float *pair_lut, int n_centroids,
                       tq4_stream_t stream);

/*
 * Full decode step: rotate query into q_rot_ws, build the pair LUT into
 * pair_lut_ws (512 floats), Stage1 into mid_o, Stage2 into out / lse; sinks as in
 * tq4_stage1_ex (may be NULL).  q_rot_ws, pair_lut_ws and mid_o are workspaces: when
 * every (sequence, kv-head) gets one Stage1 wave the step runs one split per sequence and
 * Stage1 writes out / lse itself (mid_o unwritten), and for TQ4_BF16 / TQ4_F16 queries with
 * Hk * (waves per kv-head) dividing 8 the same launch also rotates the query (q_rot_ws and
 * pair_lut_ws unwritten).
 * Replaces: tq4_cuda_v7_full cuda/tq4_cuda_v7.cu:78-84 plus the q rotation of
 *           triton_turboquant_decode_attention reference/soa_decode_v1.py:485-643.
 */
int tq4_full_decode(const void *query, int query_dtype, const float *rot_t,
                    const float *centroids, const uint8_t *kv_cache,
                    const int32_t *block_table, const int32_t *seq_lens, float *q_rot_ws,
                    float *pair_lut_ws, float *mid_o, void *out, int out_dtype, float *lse,
                    int B, int Hq, int Hk, int D, int block_size, int max_blocks_per_seq,
                    int64_t cache_block_stride, int num_kv_splits, int layout,
                    float attn_scale, const float *sinks, tq4_stream_t stream);

/*
 * tq4_full_decode without caller workspaces: the pair LUT, the rotated queries and the
 * Stage1 rows live in a 40 MiB device array the library holds on every GPU it runs on (from
 * its load until the process ends), so the call allocates nothing -- no hipMalloc, no
 * allocator.  Shapes whose workspace exceeds the array (2 KiB LUT + B*Hq*D*4 bytes of
 * q_rot + B*Hq*S*(D+1)*4 bytes of Stage1 rows unless one split per sequence applies) are
 * rejected with TQ4_E_INVALID.  Calls that overlap on one GPU share the array and race:
 * serialize them (one stream, or events).  Otherwise as tq4_full_decode.
 * No counterpart in the reference: for callers that cannot allocate (code under graph
 * capture, tight serving loops, harnesses that forbid allocation).
 */
int tq4_full_decode_noalloc(const void *query, int query_dtype, const float *rot_t,
                            const float *centroids, const uint8_t *kv_cache,
                            const int32_t *block_table, const int32_t *seq_lens, void *out,
                            int out_dtype, float *lse, int B, int Hq, int Hk, int D,
                            int block_size, int max_blocks_per_seq, int64_t cache_block_stride,
                            int num_kv_splits, int layout, float attn_scale, const float *sinks,
                            tq4_stream_t stream);

/*
 * Cache writer: quantize key / value [N, Hk, D] (dtype TQ4_F32 / TQ4_BF16 / TQ4_F16,
 * contiguous, 16-byte aligned) and write token i into cache slot slot_mapping[i]
 * (block slot / block_size, position slot % block_size; slots < 0 are skipped).  K:
 * norm, x_hat = k / (norm + 1e-8), y = x_hat @ rot_t (rot_t = PiT, [D, D] fp32), 4-bit
 * index = number of the 15 midpoints <= y, stored scalar fp16(norm / ||c[idx]||) when
 * norm_correction is nonzero (centroids [16] required), else fp16(norm).  V: 4-bit
 * uniform codes with fp16 scale and fp16 min.  layout TQ4_LAYOUT_SOA, TQ4_LAYOUT_AOS or
 * TQ4_LAYOUT_AOS_HEAD_MAJOR.
 * Replaces: triton_turboquant_store reference/soa_store.py:381-524 (MSE path, 4-bit keys
 *           and values; kernel :223-380) and the AoS writer reference/aos_store.py.
 */
int tq4_store(const void *key, const void *value, int dtype, const int32_t *slot_mapping,
              const float *rot_t, const float *midpoints, const float *centroids,
              uint8_t *kv_cache, int N, int Hk, int D, int block_size,
              int64_t cache_block_stride, int layout, int norm_correction, tq4_stream_t stream);

/*
 * FP8-key preset (turboquant_k8v4): Stage1 over a cache whose K is one OCP E4M3 byte per
 * dim (record 128 K bytes | 64 V bytes, SoA metadata fields V scale and V zero; AoS slot
 * 196 bytes = K | V | scale | zero).  query is the unrotated query (fp32 [B, Hq, D]);
 * score = q.k * attn_scale.  Same mid_o contract, grid rule and sinks as tq4_stage1_ex;
 * runs on the 16x16x32 MFMA kernel where it applies (power-of-two block_size >= 16,
 * 16-byte block stride), else on the VALU kernel.
 * Replaces: _tq_decode_stage1 with KEY_FP8=1, reference/soa_decode_v1.py:213-230 (launch
 *           :519-606); the AoS kernel reference/aos_decode.py.
 */
int tq4_stage1_fp8(const float *query, const uint8_t *kv_cache, const int32_t *block_table,
                   const int32_t *seq_lens, float *mid_o, int B, int Hq, int Hk, int D, int block_size,
                   int max_blocks_per_seq, int64_t cache_block_stride, int num_kv_splits, int layout,
                   float attn_scale, const float *sinks, tq4_stream_t stream);

/* tq4_stage1_fp8 with the kernel choice of tq4_stage1_ex (AUTO, SIMPLE or XDL).  Replaces: the same reference entry as tq4_stage1_fp8. */
int tq4_stage1_fp8_ex(const float *query, const uint8_t *kv_cache, const int32_t *block_table,
                      const int32_t *seq_lens, float *mid_o, int B, int Hq, int Hk, int D, int block_size,
                      int max_blocks_per_seq, int64_t cache_block_stride, int num_kv_splits, int layout,
                      float attn_scale, const float *sinks, int kernel, tq4_stream_t stream);

/*
 * FP8-key preset writer: K cast to E4M3 (round to nearest even, saturating at +-448, NaN
 * kept), V as tq4_store; layout as tq4_store; slots < 0 skipped.
 * Replaces: _tq_fused_store_fp8 reference/soa_store.py:125-212 (launch :446-478) and the
 *           AoS FP8 store of reference/aos_store.py.
 */
int tq4_store_fp8(const void *key, const void *value, int dtype, const int32_t *slot_mapping,
                  uint8_t *kv_cache, int N, int Hk, int D, int block_size, int64_t cache_block_stride,
                  int layout, tq4_stream_t stream);

/*
 * Bit-width presets: turboquant_k3v4_nc (key_bits 3, value_bits 4), turboquant_3bit_nc
 * (3, 3) and the 4-bit layout (4, 4), reference/config.py:20-40.  Codes are packed at
 * key_bits (value_bits) bits per dim, least significant bit first (code d at bits
 * [b*d, b*d + b) of the row).  SoA record 16*key_bits + 16*value_bits bytes with the three
 * fp16 metadata fields K norm (folded norm correction), V scale, V zero; AoS slot
 * K | fp16 norm | V | fp16 scale | fp16 zero padded to even (118 bytes for 3/4, 102 for 3/3).
 * centroids: the 2^key_bits Lloyd-Max centroids.  Same mid_o contract, grid rule and sinks
 * as tq4_stage1_ex; 3/4 and 3/3 run on the 16x16x32 MFMA kernel where it applies
 * (power-of-two block_size >= 16, 16-byte block stride), everything else on the VALU kernel.
 * Replaces: _tq_decode_stage1 with MSE_BITS = 3 / VQB = 3, reference/soa_decode_v1.py:122-132
 *           (3-bit K unpack) and :271-284 (3-bit V unpack); the AoS kernel
 *           reference/aos_decode.py:121-285.
 */
int tq4_stage1_preset(const float *q_rot, const uint8_t *kv_cache, const int32_t *block_table,
                      const int32_t *seq_lens, const float *centroids, float *mid_o, int B, int Hq,
                      int Hk, int D, int block_size, int max_blocks_per_seq,
                      int64_t cache_block_stride, int num_kv_splits, int layout, float attn_scale,
                      const float *sinks, int key_bits, int value_bits, tq4_stream_t stream);

/* tq4_stage1_preset with the kernel choice of tq4_stage1_ex (AUTO, SIMPLE, or XDL for 3/4, 3/3).
 * Replaces: the same reference entry as tq4_stage1_preset. */
int tq4_stage1_preset_ex(const float *q_rot, const uint8_t *kv_cache, const int32_t *block_table,
                         const int32_t *seq_lens, const float *centroids, float *mid_o, int B, int Hq,
                         int Hk, int D, int block_size, int max_blocks_per_seq,
                         int64_t cache_block_stride, int num_kv_splits, int layout, float attn_scale,
                         const float *sinks, int key_bits, int value_bits, int kernel,
                         tq4_stream_t stream);

/*
 * Writer of the bit-width presets (layout as tq4_stage1_preset): K index = number of the
 * 2^key_bits - 1 midpoints <= y, V scale = max((max - min) / (2^value_bits - 1), 1e-8);
 * otherwise as tq4_store (4/4 is tq4_store itself).
 * Replaces: triton_turboquant_store with MSE bits 3 / value bits 3,
 *           reference/soa_store.py:300-340 (3-bit K pack) and :47-83 (3-bit V pack); the AoS
 *           writer reference/aos_store.py.
 */
int tq4_store_preset(const void *key, const void *value, int dtype, const int32_t *slot_mapping,
                     const float *rot_t, const float *midpoints, const float *centroids,
                     uint8_t *kv_cache, int N, int Hk, int D, int block_size,
                     int64_t cache_block_stride, int layout, int norm_correction, int key_bits,
                     int value_bits, tq4_stream_t stream);

/* Message of the last failed call on this thread ("" when none).
 * Replaces: the TORCH_CHECK messages of cuda/tq4_cuda_v1.cu:468-499. */
const char *tq4_last_error(void);

/* ABI version of this library (major*100 + minor): 106 adds TQ4_LAYOUT_AOS_HEAD_MAJOR and
 * retires TQ4_KERNEL_MFMA. */
int tq4_abi_version(void);

/*
 * Measurement hook: the next kernel launch made by this thread stamps start_event and
 * stop_event (hipEvent_t, created by the caller; either may be NULL) with that kernel's
 * own start and end (hipExtLaunchKernel), the interval rocprofv3 reports as its
 * duration; the hook then clears itself.  An entry point that launches several kernels
 * (tq4_full_decode) stamps the first.  No counterpart in the reference: for benchmarks.
 */
int tq4_time_next_launch(void *start_event, void *stop_event);

#ifdef __cplusplus
}
#endif

#endif /* TQ4_DECODE_H */
