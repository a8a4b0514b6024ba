// C ABI of the gfx950 TurboQuant 4-bit decode path (declared in include/tq4_decode.h).
//
// Argument checks mirror the TORCH_CHECKs of the reference CUDA entry points
// (cuda/tq4_cuda_v1.cu:468-499, cuda/tq4_cuda_v7.cu:58-68) and the launcher asserts of
// baseline/triton_v2.py:594-607, but report through a return code and a thread-local
// message instead of throwing.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <atomic>
#include <cstdarg>
#include <mutex>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "../../include/tq4_decode.h"
#include "stage1_simple.h"
#include "stage1_xdl.h"
#include "stage2.h"
#include "store.h"

namespace {

thread_local char g_err[512] = "";

// Events the next kernel launch of this thread stamps with its own start and end
// (tq4_time_next_launch); cleared by that launch.
thread_local hipEvent_t g_time_start = nullptr, g_time_stop = nullptr;

// Every kernel launch goes through here: arguments are converted to the kernel's
// parameter types (the event-stamping launch passes them by address).
template <typename... KArgs, typename... Args>
void launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, hipStream_t st, Args... args) {
    static_assert(sizeof...(KArgs) == sizeof...(Args), "argument count");
    if (g_time_start || g_time_stop) {
        const hipEvent_t a = g_time_start, b = g_time_stop;
        g_time_start = g_time_stop = nullptr;
        hipExtLaunchKernelGGL(kernel, grid, block, 0, st, a, b, 0, static_cast<KArgs>(args)...);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, 0, st, static_cast<KArgs>(args)...);
    }
}

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int ok() {
    g_err[0] = '\0';
    return TQ4_OK;
}

int launch_status(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail((int)e, "%s launch failed: %s", what, hipGetErrorString(e));
    return ok();
}

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int log2_int(int x) {
    int r = 0;
    while ((1 << r) < x)
        ++r;
    return r;
}

struct Stage1Args {
    const float *q_rot;
    const uint8_t *cache;
    const int32_t *bt;
    const int32_t *seq_lens;
    const float *lut;
    float *mid_o;
    int B, Hq, Hk, D, bs, max_blocks;
    int64_t stride;
    int S, layout;  // TQ4_LAYOUT_*
    float scale;
    const float *sinks = nullptr;  // [Hq] sink logits of split 0, or null
    // set: one split per sequence, the XDL kernel writes the final rows (Stage2 fused)
    void *out = nullptr;
    int out_dtype = TQ4_F32;
    float *lse = nullptr;
    bool key_fp8 = false;  // the FP8-key preset (VALU kernel; pair LUT unused)
    // > 0: the key_bits / value_bits preset on the VALU kernel; lut holds the 2^key_bits
    // centroids (not the pair LUT)
    int key_bits = 0, value_bits = 4;
    // set (with out): the one-split kernel rotates this query itself (TQ4_BF16 / TQ4_F16 rows
    // [B, Hq, D]) with rot_t, and lut holds the 16 centroids instead of the pair LUT
    const void *query = nullptr;
    int query_dtype = TQ4_F32;
    const float *rot_t = nullptr;
    // filled by check_stage1: kernel layout (0 SoA, 1 AoS) and the AoS slot strides
    int kl = 0, slot_pos = 0, slot_head = 0;
};

// Kernel layout (0 SoA, 1 AoS) of an ABI layout id and the byte offsets of AoS slot (t, h)
// inside a block, t * pos + h * head: position-major blocks [bs][Hk][slot] (TQ4_LAYOUT_AOS)
// or head-major blocks [Hk][bs][slot] (TQ4_LAYOUT_AOS_HEAD_MAJOR, the layout the vLLM
// backend's [blocks, Hk, bs, slot] cache presents through transpose(1, 2),
// reference/turboquant_attn.py:536, :565).  SoA blocks are addressed by their own layout.
struct CacheGeom {
    int kl, pos, head;
};
bool layout_valid(int layout) {
    return layout == TQ4_LAYOUT_SOA || layout == TQ4_LAYOUT_AOS || layout == TQ4_LAYOUT_AOS_HEAD_MAJOR;
}
CacheGeom cache_geom(int layout, int bs, int hk, int slot) {
    if (layout == TQ4_LAYOUT_AOS_HEAD_MAJOR)
        return {1, slot, bs * slot};
    return {layout == TQ4_LAYOUT_AOS ? 1 : 0, hk * slot, slot};
}
#define TQ4_LAYOUT_MSG "layout must be 0 (SoA), 1 (AoS) or 2 (AoS, head-major blocks)"

// Bytes of one AoS slot (= SoA bytes per (token, kv-head)) of a key_bits / value_bits preset.
int preset_slot_bytes(int key_bits, int value_bits) {
    const int raw = 16 * key_bits + 2 + 16 * value_bits + 4;
    return raw + raw % 2;
}

bool preset_supported(int key_bits, int value_bits) {
    return (key_bits == 4 && value_bits == 4) || (key_bits == 3 && (value_bits == 3 || value_bits == 4));
}
static_assert(tq4::kOutF32 == TQ4_F32 && tq4::kOutBf16 == TQ4_BF16 && tq4::kOutF16 == TQ4_F16,
              "output type ids");

int check_stage1(Stage1Args &a) {
    if (!a.q_rot || !a.cache || !a.bt || !a.seq_lens || (!a.lut && !a.key_fp8) || !a.mid_o)
        return fail(TQ4_E_INVALID, "tq4_stage1: null pointer argument");
    if (a.B <= 0 || a.Hq <= 0 || a.Hk <= 0 || a.S <= 0 || a.bs <= 0 || a.max_blocks <= 0)
        return fail(TQ4_E_INVALID, "tq4_stage1: B, Hq, Hk, num_kv_splits, block_size and "
                                   "max_blocks_per_seq must be positive");
    if (a.Hq % a.Hk)
        return fail(TQ4_E_INVALID, "tq4_stage1: Hq (%d) must be a multiple of Hk (%d)", a.Hq, a.Hk);
    if (a.S > 65536)
        return fail(TQ4_E_UNSUPPORTED, "tq4_stage1: num_kv_splits %d above 65536", a.S);
    if (a.B > 65535)  // a grid dimension
        return fail(TQ4_E_UNSUPPORTED, "tq4_stage1: batch %d above 65535", a.B);
    if (a.D != tq4::kHeadDim)
        return fail(TQ4_E_UNSUPPORTED, "tq4_stage1: head_dim %d unsupported (kernels are built for 128)", a.D);
    if (!layout_valid(a.layout))
        return fail(TQ4_E_INVALID, "tq4_stage1: " TQ4_LAYOUT_MSG);
    const int slot = a.key_fp8 ? tq4::store::kFp8Record + 4
                               : (a.key_bits > 0 ? preset_slot_bytes(a.key_bits, a.value_bits) : tq4::kAosSlot);
    const int64_t min_stride = (int64_t)a.bs * a.Hk * slot;
    if (a.stride < min_stride || a.stride % 2)
        return fail(TQ4_E_INVALID, "tq4_stage1: requires cache [blocks,%d,%d,%d]: block stride %lld < %lld",
                    a.bs, a.Hk, slot, (long long)a.stride, (long long)min_stride);
    if (!aligned(a.cache, 16) || !aligned(a.q_rot, 16) || !aligned(a.mid_o, 4))
        return fail(TQ4_E_INVALID, "tq4_stage1: kv_cache and q_rot must be 16-byte aligned");
    if (!(a.scale > 0.f) || a.scale != a.scale)
        return fail(TQ4_E_INVALID, "tq4_stage1: attn_scale must be positive");
    const CacheGeom geom = cache_geom(a.layout, a.bs, a.Hk, slot);
    a.kl = geom.kl;
    a.slot_pos = geom.pos;
    a.slot_head = geom.head;
    return TQ4_OK;
}

template <int LAYOUT, int G> void launch_simple(const Stage1Args &a, hipStream_t st) {
    const dim3 grid(a.S, a.Hk, a.B);
    auto kernel = &tq4::stage1_simple_kernel<LAYOUT, G, false>;
    if (a.key_fp8)
        kernel = &tq4::stage1_simple_kernel<LAYOUT, G, true>;
    else if (a.key_bits == 4)
        kernel = &tq4::stage1_simple_kernel<LAYOUT, G, false, 4, 4>;
    else if (a.key_bits == 3 && a.value_bits == 4)
        kernel = &tq4::stage1_simple_kernel<LAYOUT, G, false, 3, 4>;
    else if (a.key_bits == 3)
        kernel = &tq4::stage1_simple_kernel<LAYOUT, G, false, 3, 3>;
    launch(kernel, grid, dim3(tq4::kWave), st,
                       a.q_rot, a.cache, a.bt, a.seq_lens, a.lut, a.mid_o, a.sinks, a.Hq, a.Hk, a.bs,
                       a.max_blocks, a.stride, a.slot_pos, a.slot_head, a.S, a.scale * tq4::kLog2e);
}

// q-heads per wave of the 16x16x32 kernel (4 for GQA groups up to 4, else 8) and the waves
// (parts) each kv-head's group takes.
int xdl_heads(const Stage1Args &a) { return a.Hq / a.Hk <= 4 ? 4 : 8; }
int xdl_parts(const Stage1Args &a) {
    const int g = a.Hq / a.Hk, h = xdl_heads(a);
    return (g + h - 1) / h;
}

// Waves per (sequence, kv-head part) for the 16x16x32 kernel; wave x takes splits
// [x * S / W, (x + 1) * S / W).  Consecutive splits in one wave share one load
// pipeline, which removes per-split start-up latency; W is chosen so the grid fills
// whole rounds of the waves the GPU holds at the kernel's occupancy.  `slots` caches that
// count per kernel instance (computed on the first call; concurrent first calls compute the
// same value).  TQ4_STAGE1_WAVES overrides W (a tuning knob; results do not depend on it).
int waves_per_sequence(const Stage1Args &a, const void *kernel, std::atomic<int> &slots) {
    static const int forced = [] {
        const char *e = getenv("TQ4_STAGE1_WAVES");
        return e ? atoi(e) : 0;
    }();
    if (forced > 0)
        return forced < a.S ? forced : a.S;
    int held = slots.load(std::memory_order_relaxed);
    if (!held) {  // waves the device holds at once for this kernel
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, tq4::kWave, 0) == hipSuccess &&
            cus > 0 && per_cu > 0)
            held = cus * per_cu;
        else
            held = 256 * 4 * 2;
        slots.store(held, std::memory_order_relaxed);
    }
    const int64_t pairs = (int64_t)a.Hk * xdl_parts(a) * a.B;
    // smallest number of whole rounds that gives every pair at least one wave
    const int64_t rounds = (pairs + held - 1) / held;
    int64_t w = rounds * held / pairs;
    if (w < 1)
        w = 1;
    return (int)(w < a.S ? w : a.S);
}

// Waves per SIMD the 16x16x32 kernel is built for.  Two: the SoA G=4 kernel also fits
// three (168 VGPRs, a 5-split LDS image), but runs slower that way.
#ifndef TQ4_XDL_WAVES_PER_SIMD
#define TQ4_XDL_WAVES_PER_SIMD 2
#endif
template <int LAYOUT, int G> constexpr int xdl_waves_per_simd() {
    return LAYOUT == 0 && G == 4 ? TQ4_XDL_WAVES_PER_SIMD : 2;
}

template <int LAYOUT, int G, bool KF8 = false, bool KB3 = false, bool V3 = false> int xdl_waves(const Stage1Args &a) {
    static std::atomic<int> slots{0};
    const auto kernel = &tq4::xdl::stage1_xdl_kernel<LAYOUT, G, xdl_waves_per_simd<LAYOUT, G>(), false, KF8, KB3, V3>;
    return waves_per_sequence(a, reinterpret_cast<const void *>(kernel), slots);
}

// The one-split kernel that rotates the query itself: one workgroup per sequence holding its
// Hk * parts waves, which must divide 8 (two waves per SIMD of one CU).
bool rot_applies(const Stage1Args &a) {
    const int nvh = a.Hk * xdl_parts(a);
    return (a.query_dtype == TQ4_BF16 || a.query_dtype == TQ4_F16) && 8 % nvh == 0;
}

template <int LAYOUT, int G> void launch_xdl(const Stage1Args &a, hipStream_t st) {
    constexpr int wpe = xdl_waves_per_simd<LAYOUT, G>();
    const bool kb3 = a.key_bits == 3, v3 = a.value_bits == 3;
    const int nvh = a.Hk * xdl_parts(a);
    if (a.query) {  // one split per sequence, the rotation inside (Stage2 fused)
        const auto kernel = a.query_dtype == TQ4_BF16
                                ? &tq4::xdl::stage1_xdl_kernel<LAYOUT, G, wpe, true, false, false, false, 1>
                                : &tq4::xdl::stage1_xdl_kernel<LAYOUT, G, wpe, true, false, false, false, 2>;
        launch(kernel, dim3(a.B), dim3(tq4::kWave * nvh), st, a.q_rot, a.cache, a.bt, a.seq_lens, a.lut,
               a.mid_o, a.sinks, a.out, a.out_dtype, a.lse, a.Hq, a.Hk, log2_int(a.bs), a.max_blocks,
               a.stride, a.slot_pos, a.slot_head, a.S, a.scale * tq4::kLog2e, a.query, a.rot_t);
        return;
    }
    const int waves = a.key_fp8 ? xdl_waves<LAYOUT, G, true>(a)
                      : kb3     ? (v3 ? xdl_waves<LAYOUT, G, false, true, true>(a) : xdl_waves<LAYOUT, G, false, true>(a))
                                : xdl_waves<LAYOUT, G>(a);
    const dim3 grid(nvh, waves, a.B);
    auto kernel = a.out ? &tq4::xdl::stage1_xdl_kernel<LAYOUT, G, wpe, true>
                        : &tq4::xdl::stage1_xdl_kernel<LAYOUT, G, wpe, false>;
    if (a.key_fp8)  // never fused: the FP8-key decode runs Stage2 itself
        kernel = &tq4::xdl::stage1_xdl_kernel<LAYOUT, G, wpe, false, true>;
    else if (kb3)  // 3-bit keys, 4- or 3-bit values; never fused
        kernel = v3 ? &tq4::xdl::stage1_xdl_kernel<LAYOUT, G, wpe, false, false, true, true>
                    : &tq4::xdl::stage1_xdl_kernel<LAYOUT, G, wpe, false, false, true>;
    launch(kernel, grid, dim3(tq4::kWave), st, a.q_rot, a.cache, a.bt, a.seq_lens, a.lut,
           a.mid_o, a.sinks, a.out, a.out_dtype, a.lse, a.Hq, a.Hk, log2_int(a.bs), a.max_blocks,
           a.stride, a.slot_pos, a.slot_head, a.S, a.scale * tq4::kLog2e, nullptr, nullptr);
}

template <int LAYOUT> int dispatch_simple(const Stage1Args &a, hipStream_t st) {
    switch (a.Hq / a.Hk) {
    case 1: launch_simple<LAYOUT, 1>(a, st); break;
    case 2: launch_simple<LAYOUT, 2>(a, st); break;
    case 4: launch_simple<LAYOUT, 4>(a, st); break;
    case 6: launch_simple<LAYOUT, 6>(a, st); break;
    case 8: launch_simple<LAYOUT, 8>(a, st); break;
    case 16: launch_simple<LAYOUT, 16>(a, st); break;
    default:
        return fail(TQ4_E_UNSUPPORTED, "tq4_stage1: GQA group %d unsupported (1, 2, 4, 6, 8, 16)",
                    a.Hq / a.Hk);
    }
    return launch_status("stage1_simple");
}

// Every GQA group: groups up to 4 on 4-head waves (1, 2 and 3 with padding heads: each KV
// tile is still read and looked up once per wave, so MHA and GQA-2 take about the headline's
// time, 1.4-1.5x faster than the VALU kernel), larger ones in parts of 8 heads (6: one part
// with two padding heads; 16: two parts).
bool mfma_applies(const Stage1Args &a) {
    const bool pow2 = a.bs >= 16 && (a.bs & (a.bs - 1)) == 0;
    return pow2 && a.stride % 16 == 0;
}

template <int LAYOUT> int dispatch_xdl(const Stage1Args &a, hipStream_t st) {
    if (!mfma_applies(a))
        return fail(TQ4_E_UNSUPPORTED, "tq4_stage1: XDL kernel needs a power-of-two block_size >= 16 "
                                       "and a 16-byte block stride");
    if (xdl_heads(a) == 4)
        launch_xdl<LAYOUT, 4>(a, st);
    else
        launch_xdl<LAYOUT, 8>(a, st);
    return launch_status("stage1_xdl");
}

// Waves per (sequence, kv-head) the auto Stage1 kernel runs with (0 when it is not the
// 16x16x32 kernel).
int auto_xdl_waves(const Stage1Args &a) {
    if (!mfma_applies(a))
        return 0;
    const bool g4 = xdl_heads(a) == 4;
    if (a.kl == 0)
        return g4 ? xdl_waves<0, 4>(a) : xdl_waves<0, 8>(a);
    return g4 ? xdl_waves<1, 4>(a) : xdl_waves<1, 8>(a);
}

int run_stage1(Stage1Args a, int kernel, hipStream_t st) {
    int rc = check_stage1(a);
    if (rc)
        return rc;
    // AUTO: the 16x16x32 kernel wherever it applies (both layouts), else VALU.
    if (kernel == TQ4_KERNEL_MFMA)
        return fail(TQ4_E_UNSUPPORTED, "tq4_stage1_ex: the 4x4x4 MFMA kernel is retired; "
                                       "TQ4_KERNEL_XDL (16x16x32) covers the same shapes");
    if (a.key_fp8 && a.out)
        return fail(TQ4_E_UNSUPPORTED, "tq4_stage1_fp8: no fused Stage2 for FP8 keys");
    // the bit-width presets: 3-bit K (4- or 3-bit V) also on the 16x16x32 kernel, 4/4 VALU
    const bool preset_xdl = a.key_bits == 3;
    if (a.key_bits > 0 && kernel != TQ4_KERNEL_AUTO && kernel != TQ4_KERNEL_SIMPLE &&
        !(preset_xdl && kernel == TQ4_KERNEL_XDL))
        return fail(TQ4_E_UNSUPPORTED, "tq4_stage1_preset: key/value bits %d/%d run on the VALU kernel%s",
                    a.key_bits, a.value_bits, preset_xdl ? " or the 16x16x32 kernel" : "");
    if (a.key_bits > 0 && a.out)
        return fail(TQ4_E_UNSUPPORTED, "tq4_stage1_preset: no fused Stage2 for the bit-width presets");
    if (kernel == TQ4_KERNEL_AUTO)
        kernel = (a.key_bits > 0 && !preset_xdl) ? TQ4_KERNEL_SIMPLE
                                                 : (mfma_applies(a) ? TQ4_KERNEL_XDL : TQ4_KERNEL_SIMPLE);
    if (kernel == TQ4_KERNEL_SIMPLE)
        return a.kl == 0 ? dispatch_simple<0>(a, st) : dispatch_simple<1>(a, st);
    if (kernel == TQ4_KERNEL_XDL)
        return a.kl == 0 ? dispatch_xdl<0>(a, st) : dispatch_xdl<1>(a, st);
    return fail(TQ4_E_INVALID, "tq4_stage1_ex: unknown kernel id %d", kernel);
}

int rotate_query(const void *query, int query_dtype, const float *rot_t, float *q_rot, int rows,
                 int D, const float *centroids, float *pair_lut, hipStream_t st) {
    if (!query || !rot_t || !q_rot)
        return fail(TQ4_E_INVALID, "tq4_rotate_query: null pointer argument");
    if (rows <= 0)
        return fail(TQ4_E_INVALID, "tq4_rotate_query: rows must be positive");
    if (D != tq4::kHeadDim)
        return fail(TQ4_E_UNSUPPORTED, "tq4_rotate_query: head_dim %d unsupported (128)", D);
    if (!aligned(query, 16))
        return fail(TQ4_E_INVALID, "tq4_rotate_query: query must be 16-byte aligned");
    const dim3 grid((rows + tq4::kRotMfmaRows - 1) / tq4::kRotMfmaRows), block(tq4::kWave * tq4::kRotWaves);
    switch (query_dtype) {
    case TQ4_F32:
        launch(&tq4::rotate_mfma_kernel<float>, grid, block, st,
                           static_cast<const float *>(query), rot_t, q_rot, rows, centroids, pair_lut);
        break;
    case TQ4_BF16:
        launch(&tq4::rotate_mfma_kernel<__bf16>, grid, block, st,
                           static_cast<const __bf16 *>(query), rot_t, q_rot, rows, centroids, pair_lut);
        break;
    case TQ4_F16:
        launch(&tq4::rotate_mfma_kernel<_Float16>, grid, block, st,
                           static_cast<const _Float16 *>(query), rot_t, q_rot, rows, centroids, pair_lut);
        break;
    default:
        return fail(TQ4_E_INVALID, "tq4_rotate_query: query_dtype must be 0, 1 or 2");
    }
    return launch_status("rotate_query");
}

// The writer for KB-bit K indices / VB-bit V codes over `rows` (token, kv-head) rows.
template <int KB, int VB>
int launch_store(const void *key, const void *value, int dtype, const int32_t *slot_mapping,
                 const float *rot_t, const float *midpoints, const float *centroids, uint8_t *kv_cache,
                 int rows, int Hk, int block_size, int64_t cache_block_stride, const CacheGeom &geom,
                 int norm_correction, hipStream_t st, const char *what) {
    // few tiles: 4-wave workgroups, one per CU at most (see store_kernel)
    const int64_t tiles = ((int64_t)rows + tq4::store::kRows - 1) / tq4::store::kRows;
    const bool small = tiles <= tq4::store::kSmallTiles;
    const int waves = small ? tq4::store::kSmallWaves : tq4::store::kWaves;
    const dim3 grid(std::min<int64_t>((tiles + waves - 1) / waves, tq4::store::kMaxGroups));
#define TQ4_STORE_LAUNCH(L, T)                                                                             \
    (small ? launch(&tq4::store::store_kernel<L, T, KB, VB, tq4::store::kSmallWaves>, grid,               \
                    dim3(tq4::kWave * tq4::store::kSmallWaves), st, static_cast<const T *>(key),            \
                    static_cast<const T *>(value), slot_mapping, rot_t, midpoints, centroids, kv_cache,     \
                    rows, Hk, block_size, cache_block_stride, geom.pos, geom.head, norm_correction)         \
           : launch(&tq4::store::store_kernel<L, T, KB, VB>, grid, dim3(tq4::kWave * tq4::store::kWaves),   \
                    st, static_cast<const T *>(key), static_cast<const T *>(value), slot_mapping, rot_t,    \
                    midpoints, centroids, kv_cache, rows, Hk, block_size, cache_block_stride, geom.pos,     \
                    geom.head, norm_correction))
    switch (dtype * 2 + geom.kl) {
    case TQ4_F32 * 2 + 0: TQ4_STORE_LAUNCH(0, float); break;
    case TQ4_F32 * 2 + 1: TQ4_STORE_LAUNCH(1, float); break;
    case TQ4_BF16 * 2 + 0: TQ4_STORE_LAUNCH(0, __bf16); break;
    case TQ4_BF16 * 2 + 1: TQ4_STORE_LAUNCH(1, __bf16); break;
    case TQ4_F16 * 2 + 0: TQ4_STORE_LAUNCH(0, _Float16); break;
    case TQ4_F16 * 2 + 1: TQ4_STORE_LAUNCH(1, _Float16); break;
    default:
        return fail(TQ4_E_INVALID, "%s: dtype must be 0 (f32), 1 (bf16) or 2 (f16)", what);
    }
#undef TQ4_STORE_LAUNCH
    return launch_status(what);
}

// Workspace of tq4_full_decode_noalloc in device memory the library owns: the pair LUT,
// the rotated queries and (unless one split per sequence applies) the Stage1 rows.  One
// copy per GPU the library runs on, held from the code object's load until the process
// ends; calls that overlap on one GPU share it and race.  Nothing in it has to start at
// zero: the rotation launch writes the LUT and q_rot before Stage1 reads them, and Stage2
// reads only the rows of non-empty splits, which Stage1 writes.
constexpr size_t kScratchBytes = size_t(40) << 20;
constexpr size_t kScratchAlign = 256;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

// Device address of `scratch` on the current device, looked up once per device (the host
// symbol is only a handle for the lookup).
constexpr int kMaxDevices = 64;
std::atomic<void *> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

int scratch_address(void **ptr) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return fail((int)e, "tq4_full_decode_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(TQ4_E_UNSUPPORTED, "tq4_full_decode_noalloc: device %d beyond the %d the library tracks", dev,
                    kMaxDevices);
    void *p = g_scratch[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch[dev].load(std::memory_order_relaxed);
        if (!p) {
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !p)
                return fail(e != hipSuccess ? (int)e : TQ4_E_INVALID,
                            "tq4_full_decode_noalloc: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
            g_scratch[dev].store(p, std::memory_order_release);
        }
    }
    *ptr = p;
    return TQ4_OK;
}

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

}  // namespace

extern "C" {

int tq4_time_next_launch(void *start_event, void *stop_event) {
    g_time_start = reinterpret_cast<hipEvent_t>(start_event);
    g_time_stop = reinterpret_cast<hipEvent_t>(stop_event);
    return ok();
}

int tq4_abi_version(void) { return 106; }

const char *tq4_last_error(void) { return g_err; }

int tq4_stage1_ex(const float *q_rot, const uint8_t *kv_cache, const int32_t *block_table,
                  const int32_t *seq_lens, const float *pair_lut, float *mid_o, int B, int Hq,
                  int Hk, int D, int block_size, int max_blocks_per_seq,
                  int64_t cache_block_stride, int num_kv_splits, int layout, float attn_scale,
                  int kernel, const float *sinks, tq4_stream_t stream) {
    const Stage1Args a{q_rot, kv_cache, block_table, seq_lens, pair_lut, mid_o, B, Hq, Hk, D,
                       block_size, max_blocks_per_seq, cache_block_stride, num_kv_splits,
                       layout, attn_scale, sinks};
    return run_stage1(a, kernel, reinterpret_cast<hipStream_t>(stream));
}

int tq4_stage1(const float *q_rot, const uint8_t *kv_cache, const int32_t *block_table,
               const int32_t *seq_lens, const float *pair_lut, float *mid_o, int B, int Hq,
               int Hk, int D, int block_size, int max_blocks_per_seq,
               int64_t cache_block_stride, int num_kv_splits, int layout, float attn_scale,
               tq4_stream_t stream) {
    return tq4_stage1_ex(q_rot, kv_cache, block_table, seq_lens, pair_lut, mid_o, B, Hq, Hk, D,
                         block_size, max_blocks_per_seq, cache_block_stride, num_kv_splits,
                         layout, attn_scale, TQ4_KERNEL_AUTO, nullptr, stream);
}

int tq4_stage1_fp8_ex(const float *query, const uint8_t *kv_cache, const int32_t *block_table,
                      const int32_t *seq_lens, float *mid_o, int B, int Hq, int Hk, int D, int block_size,
                      int max_blocks_per_seq, int64_t cache_block_stride, int num_kv_splits, int layout,
                      float attn_scale, const float *sinks, int kernel, tq4_stream_t stream) {
    Stage1Args a{query, kv_cache, block_table, seq_lens, nullptr, mid_o, B, Hq, Hk, D,
                 block_size, max_blocks_per_seq, cache_block_stride, num_kv_splits, layout,
                 attn_scale, sinks};
    a.key_fp8 = true;
    return run_stage1(a, kernel, reinterpret_cast<hipStream_t>(stream));
}

int tq4_stage1_fp8(const float *query, const uint8_t *kv_cache, const int32_t *block_table,
                   const int32_t *seq_lens, float *mid_o, int B, int Hq, int Hk, int D, int block_size,
                   int max_blocks_per_seq, int64_t cache_block_stride, int num_kv_splits, int layout,
                   float attn_scale, const float *sinks, tq4_stream_t stream) {
    return tq4_stage1_fp8_ex(query, kv_cache, block_table, seq_lens, mid_o, B, Hq, Hk, D, block_size,
                             max_blocks_per_seq, cache_block_stride, num_kv_splits, layout, attn_scale,
                             sinks, TQ4_KERNEL_AUTO, stream);
}

int tq4_stage1_preset_ex(const float *q_rot, const uint8_t *kv_cache, const int32_t *block_table,
                         const int32_t *seq_lens, const float *centroids, float *mid_o, int B, int Hq,
                         int Hk, int D, int block_size, int max_blocks_per_seq,
                         int64_t cache_block_stride, int num_kv_splits, int layout, float attn_scale,
                         const float *sinks, int key_bits, int value_bits, int kernel,
                         tq4_stream_t stream) {
    if (!preset_supported(key_bits, value_bits))
        return fail(TQ4_E_UNSUPPORTED, "tq4_stage1_preset: key_bits / value_bits %d / %d unsupported "
                                       "(4/4, 3/4, 3/3)", key_bits, value_bits);
    Stage1Args a{q_rot, kv_cache, block_table, seq_lens, centroids, mid_o, B, Hq, Hk, D,
                 block_size, max_blocks_per_seq, cache_block_stride, num_kv_splits, layout,
                 attn_scale, sinks};
    a.key_bits = key_bits;
    a.value_bits = value_bits;
    return run_stage1(a, kernel, reinterpret_cast<hipStream_t>(stream));
}

int tq4_stage1_preset(const float *q_rot, const uint8_t *kv_cache, const int32_t *block_table,
                      const int32_t *seq_lens, const float *centroids, float *mid_o, int B, int Hq,
                      int Hk, int D, int block_size, int max_blocks_per_seq,
                      int64_t cache_block_stride, int num_kv_splits, int layout, float attn_scale,
                      const float *sinks, int key_bits, int value_bits, tq4_stream_t stream) {
    return tq4_stage1_preset_ex(q_rot, kv_cache, block_table, seq_lens, centroids, mid_o, B, Hq, Hk, D,
                                block_size, max_blocks_per_seq, cache_block_stride, num_kv_splits, layout,
                                attn_scale, sinks, key_bits, value_bits, TQ4_KERNEL_AUTO, stream);
}

int tq4_stage2(const float *mid_o, const int32_t *seq_lens, void *out, int out_dtype,
               float *lse, int B, int Hq, int D, int num_kv_splits, tq4_stream_t stream) {
    if (!mid_o || !seq_lens || !out || !lse)
        return fail(TQ4_E_INVALID, "tq4_stage2: null pointer argument");
    if (B <= 0 || Hq <= 0 || num_kv_splits <= 0)
        return fail(TQ4_E_INVALID, "tq4_stage2: B, Hq and num_kv_splits must be positive");
    if (D != tq4::kHeadDim)
        return fail(TQ4_E_UNSUPPORTED, "tq4_stage2: head_dim %d unsupported (128)", D);
    if (num_kv_splits > 65536 || B > 65535)
        return fail(TQ4_E_UNSUPPORTED, "tq4_stage2: num_kv_splits %d above 65536 or batch %d above 65535",
                    num_kv_splits, B);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const dim3 grid(Hq, B);
    switch (out_dtype) {
    case TQ4_F32:
        launch(&tq4::stage2_kernel<float>, grid, dim3(tq4::kWave), st, mid_o,
                           seq_lens, static_cast<float *>(out), lse, Hq, num_kv_splits);
        break;
    case TQ4_BF16:
        launch(&tq4::stage2_kernel<__bf16>, grid, dim3(tq4::kWave), st, mid_o,
                           seq_lens, static_cast<__bf16 *>(out), lse, Hq, num_kv_splits);
        break;
    case TQ4_F16:
        launch(&tq4::stage2_kernel<_Float16>, grid, dim3(tq4::kWave), st, mid_o,
                           seq_lens, static_cast<_Float16 *>(out), lse, Hq, num_kv_splits);
        break;
    default:
        return fail(TQ4_E_INVALID, "tq4_stage2: out_dtype must be 0 (f32), 1 (bf16) or 2 (f16)");
    }
    return launch_status("stage2");
}

int tq4_rotate_query(const void *query, int query_dtype, const float *rot_t, float *q_rot,
                     int rows, int D, tq4_stream_t stream) {
    return rotate_query(query, query_dtype, rot_t, q_rot, rows, D, nullptr, nullptr,
                        reinterpret_cast<hipStream_t>(stream));
}

int tq4_build_pair_lut(const float *centroids, float *pair_lut, int n_centroids,
                       tq4_stream_t stream) {
    if (!centroids || !pair_lut)
        return fail(TQ4_E_INVALID, "tq4_build_pair_lut: null pointer argument");
    if (n_centroids != 16)
        return fail(TQ4_E_UNSUPPORTED, "tq4_build_pair_lut: 16 centroids (4-bit keys) expected, got %d",
                    n_centroids);
    launch(&tq4::pair_lut_kernel, dim3(1), dim3(256), reinterpret_cast<hipStream_t>(stream), centroids,
           pair_lut, n_centroids);
    return launch_status("pair_lut");
}

int tq4_full_decode(const void *query, int query_dtype, const float *rot_t,
                    const float *centroids, const uint8_t *kv_cache,
                    const int32_t *block_table, const int32_t *seq_lens, float *q_rot_ws,
                    float *pair_lut_ws, float *mid_o, void *out, int out_dtype, float *lse,
                    int B, int Hq, int Hk, int D, int block_size, int max_blocks_per_seq,
                    int64_t cache_block_stride, int num_kv_splits, int layout,
                    float attn_scale, const float *sinks, tq4_stream_t stream) {
    if (!centroids || !pair_lut_ws)
        return fail(TQ4_E_INVALID, "tq4_full_decode: null pointer argument");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    // When the Stage1 kernel gives each (sequence, kv-head part) one wave anyway, that wave
    // runs the whole sequence as one split: the same attention (up to rounding), without
    // writing and re-reading num_kv_splits rows per head (with sinks too: the sink enters
    // split 0, the only split then).  Stage2's merge of one split is the identity, so the
    // Stage1 kernel writes the output rows and LSE itself (mid_o is not written then).
    Stage1Args a{q_rot_ws, kv_cache, block_table, seq_lens, pair_lut_ws, mid_o, B, Hq, Hk, D,
                 block_size, max_blocks_per_seq, cache_block_stride, num_kv_splits, layout,
                 attn_scale, sinks};
    a.query_dtype = query_dtype;
    if (check_stage1(a) == TQ4_OK && auto_xdl_waves(a) == 1) {
        if (!out || !lse || !query || !rot_t)
            return fail(TQ4_E_INVALID, "tq4_full_decode: null pointer argument");
        if (out_dtype != TQ4_F32 && out_dtype != TQ4_BF16 && out_dtype != TQ4_F16)
            return fail(TQ4_E_INVALID, "tq4_full_decode: out_dtype must be 0 (f32), 1 (bf16) or 2 (f16)");
        a.S = 1;
        a.out = out;
        a.out_dtype = out_dtype;
        a.lse = lse;
        if (rot_applies(a) && aligned(query, 16)) {
            // one launch: the workgroup of each sequence rotates its query into LDS (the
            // workspaces q_rot_ws and pair_lut_ws are not written)
            a.query = query;
            a.rot_t = rot_t;
            a.lut = centroids;
            return run_stage1(a, TQ4_KERNEL_XDL, st);
        }
        const int rc = rotate_query(query, query_dtype, rot_t, q_rot_ws, B * Hq, D, centroids, pair_lut_ws, st);
        return rc ? rc : run_stage1(a, TQ4_KERNEL_XDL, st);
    }
    // one launch rotates the query and writes the pair LUT
    int rc = rotate_query(query, query_dtype, rot_t, q_rot_ws, B * Hq, D, centroids, pair_lut_ws, st);
    if (rc)
        return rc;
    rc = run_stage1(a, TQ4_KERNEL_AUTO, st);
    if (rc)
        return rc;
    return tq4_stage2(mid_o, seq_lens, out, out_dtype, lse, B, Hq, D, a.S, stream);
}

int tq4_full_decode_noalloc(const void *query, int query_dtype, const float *rot_t,
                            const float *centroids, const uint8_t *kv_cache,
                            const int32_t *block_table, const int32_t *seq_lens, void *out,
                            int out_dtype, float *lse, int B, int Hq, int Hk, int D,
                            int block_size, int max_blocks_per_seq, int64_t cache_block_stride,
                            int num_kv_splits, int layout, float attn_scale, const float *sinks,
                            tq4_stream_t stream) {
    if (B <= 0 || Hq <= 0 || num_kv_splits <= 0)
        return fail(TQ4_E_INVALID, "tq4_full_decode_noalloc: B, Hq and num_kv_splits must be positive");
    if (D != tq4::kHeadDim)
        return fail(TQ4_E_UNSUPPORTED, "tq4_full_decode_noalloc: head_dim %d unsupported (128)", D);
    void *base = nullptr;
    int rc = scratch_address(&base);
    if (rc)
        return rc;
    // scratch layout: pair LUT | q_rot [B, Hq, D] | mid_o [B, Hq, S, D + 1] (only when Stage1
    // runs more than one split per sequence), each 256-byte aligned
    unsigned char *bytes = static_cast<unsigned char *>(base);
    const size_t lut_bytes = round_up(256 * 2 * sizeof(float), kScratchAlign);
    const size_t q_bytes = round_up((size_t)B * Hq * D * sizeof(float), kScratchAlign);
    float *lut = reinterpret_cast<float *>(bytes);
    float *q_rot = reinterpret_cast<float *>(bytes + lut_bytes);
    float *mid_o = reinterpret_cast<float *>(bytes + lut_bytes + q_bytes);
    Stage1Args a{q_rot, kv_cache, block_table, seq_lens, lut, mid_o, B, Hq, Hk, D, block_size,
                 max_blocks_per_seq, cache_block_stride, num_kv_splits, layout, attn_scale, sinks};
    rc = check_stage1(a);  // invalid arguments report their own error, not a workspace size
    if (rc)
        return rc;
    const bool one_split = auto_xdl_waves(a) == 1;
    const size_t mid_bytes = one_split ? 0 : (size_t)B * Hq * num_kv_splits * (D + 1) * sizeof(float);
    const size_t need = lut_bytes + q_bytes + mid_bytes;
    if (need > kScratchBytes)
        return fail(TQ4_E_INVALID,
                    "tq4_full_decode_noalloc: B=%d Hq=%d S=%d needs %zu bytes of workspace (q_rot %zu, "
                    "mid_o %zu), the library's scratch holds %zu",
                    B, Hq, num_kv_splits, need, q_bytes, mid_bytes, kScratchBytes);
    return tq4_full_decode(query, query_dtype, rot_t, centroids, kv_cache, block_table, seq_lens, q_rot, lut,
                           mid_o, out, out_dtype, lse, B, Hq, Hk, D, block_size, max_blocks_per_seq,
                           cache_block_stride, num_kv_splits, layout, attn_scale, sinks, stream);
}

int tq4_store(const void *key, const void *value, int dtype, const int32_t *slot_mapping,
              const float *rot_t, const float *midpoints, const float *centroids,
              uint8_t *kv_cache, int N, int Hk, int D, int block_size,
              int64_t cache_block_stride, int layout, int norm_correction, tq4_stream_t stream) {
    if (!key || !value || !slot_mapping || !rot_t || !midpoints || !kv_cache)
        return fail(TQ4_E_INVALID, "tq4_store: null pointer argument");
    if (norm_correction && !centroids)
        return fail(TQ4_E_INVALID, "tq4_store: norm_correction requires centroids");
    if (N < 0 || Hk <= 0 || block_size <= 0)
        return fail(TQ4_E_INVALID, "tq4_store: N must be >= 0, Hk and block_size positive");
    if (D != tq4::kHeadDim)
        return fail(TQ4_E_UNSUPPORTED, "tq4_store: head_dim %d unsupported (128)", D);
    if (!layout_valid(layout))
        return fail(TQ4_E_INVALID, "tq4_store: " TQ4_LAYOUT_MSG);
    const int64_t min_stride = (int64_t)block_size * Hk * tq4::kAosSlot;
    if (cache_block_stride < min_stride || cache_block_stride % 16)
        return fail(TQ4_E_INVALID, "tq4_store: requires cache [blocks,%d,%d,134]: block stride %lld",
                    block_size, Hk, (long long)cache_block_stride);
    if (!aligned(key, 16) || !aligned(value, 16) || !aligned(kv_cache, 16))
        return fail(TQ4_E_INVALID, "tq4_store: key, value and kv_cache must be 16-byte aligned");
    if ((int64_t)N * Hk > INT32_MAX - 64)
        return fail(TQ4_E_INVALID, "tq4_store: N * Hk = %lld rows exceeds the 32-bit row index",
                    (long long)N * Hk);
    if (N == 0)
        return ok();
    return launch_store<4, 4>(key, value, dtype, slot_mapping, rot_t, midpoints, centroids, kv_cache,
                              N * Hk, Hk, block_size, cache_block_stride,
                              cache_geom(layout, block_size, Hk, tq4::kAosSlot), norm_correction,
                              reinterpret_cast<hipStream_t>(stream), "tq4_store");
}

int tq4_store_preset(const void *key, const void *value, int dtype, const int32_t *slot_mapping,
                     const float *rot_t, const float *midpoints, const float *centroids,
                     uint8_t *kv_cache, int N, int Hk, int D, int block_size,
                     int64_t cache_block_stride, int layout, int norm_correction, int key_bits,
                     int value_bits, tq4_stream_t stream) {
    if (!preset_supported(key_bits, value_bits))
        return fail(TQ4_E_UNSUPPORTED, "tq4_store_preset: key_bits / value_bits %d / %d unsupported "
                                       "(4/4, 3/4, 3/3)", key_bits, value_bits);
    if (key_bits == 4)
        return tq4_store(key, value, dtype, slot_mapping, rot_t, midpoints, centroids, kv_cache, N, Hk, D,
                         block_size, cache_block_stride, layout, norm_correction, stream);
    if (!key || !value || !slot_mapping || !rot_t || !midpoints || !kv_cache)
        return fail(TQ4_E_INVALID, "tq4_store_preset: null pointer argument");
    if (norm_correction && !centroids)
        return fail(TQ4_E_INVALID, "tq4_store_preset: norm_correction requires centroids");
    if (N < 0 || Hk <= 0 || block_size <= 0)
        return fail(TQ4_E_INVALID, "tq4_store_preset: N must be >= 0, Hk and block_size positive");
    if (D != tq4::kHeadDim)
        return fail(TQ4_E_UNSUPPORTED, "tq4_store_preset: head_dim %d unsupported (128)", D);
    if (!layout_valid(layout))
        return fail(TQ4_E_INVALID, "tq4_store_preset: " TQ4_LAYOUT_MSG);
    const int slot = preset_slot_bytes(key_bits, value_bits);
    const int64_t min_stride = (int64_t)block_size * Hk * slot;
    if (cache_block_stride < min_stride || cache_block_stride % 2)
        return fail(TQ4_E_INVALID, "tq4_store_preset: requires cache [blocks,%d,%d,%d]: block stride %lld",
                    block_size, Hk, slot, (long long)cache_block_stride);
    if (!aligned(key, 16) || !aligned(value, 16) || !aligned(kv_cache, 2))
        return fail(TQ4_E_INVALID, "tq4_store_preset: key and value must be 16-byte aligned, kv_cache 2-byte");
    if ((int64_t)N * Hk > INT32_MAX - 64)
        return fail(TQ4_E_INVALID, "tq4_store_preset: N * Hk = %lld rows exceeds the 32-bit row index",
                    (long long)N * Hk);
    if (N == 0)
        return ok();
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const CacheGeom geom = cache_geom(layout, block_size, Hk, slot);
    if (value_bits == 4)
        return launch_store<3, 4>(key, value, dtype, slot_mapping, rot_t, midpoints, centroids, kv_cache,
                                  N * Hk, Hk, block_size, cache_block_stride, geom, norm_correction, st,
                                  "tq4_store_preset");
    return launch_store<3, 3>(key, value, dtype, slot_mapping, rot_t, midpoints, centroids, kv_cache,
                              N * Hk, Hk, block_size, cache_block_stride, geom, norm_correction, st,
                              "tq4_store_preset");
}

int tq4_store_fp8(const void *key, const void *value, int dtype, const int32_t *slot_mapping,
                  uint8_t *kv_cache, int N, int Hk, int D, int block_size, int64_t cache_block_stride,
                  int layout, tq4_stream_t stream) {
    if (!key || !value || !slot_mapping || !kv_cache)
        return fail(TQ4_E_INVALID, "tq4_store_fp8: null pointer argument");
    if (N < 0 || Hk <= 0 || block_size <= 0)
        return fail(TQ4_E_INVALID, "tq4_store_fp8: N must be >= 0, Hk and block_size positive");
    if (D != tq4::kHeadDim)
        return fail(TQ4_E_UNSUPPORTED, "tq4_store_fp8: head_dim %d unsupported (128)", D);
    if (!layout_valid(layout))
        return fail(TQ4_E_INVALID, "tq4_store_fp8: " TQ4_LAYOUT_MSG);
    const int slot = tq4::store::kFp8Record + 4;
    const int64_t min_stride = (int64_t)block_size * Hk * slot;
    if (cache_block_stride < min_stride || cache_block_stride % 4)
        return fail(TQ4_E_INVALID, "tq4_store_fp8: requires cache [blocks,%d,%d,%d]: block stride %lld",
                    block_size, Hk, slot, (long long)cache_block_stride);
    if (!aligned(key, 16) || !aligned(value, 16) || !aligned(kv_cache, 4))
        return fail(TQ4_E_INVALID, "tq4_store_fp8: key and value must be 16-byte aligned, kv_cache 4-byte");
    if ((int64_t)N * Hk > INT32_MAX - 64)
        return fail(TQ4_E_INVALID, "tq4_store_fp8: N * Hk = %lld rows exceeds the 32-bit row index",
                    (long long)N * Hk);
    if (N == 0)
        return ok();
    const int rows = N * Hk;
    const int per_group = tq4::store::kRows * tq4::store::kFp8Waves;
    const dim3 grid(std::min<int64_t>((rows + per_group - 1) / per_group, 2048));
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const CacheGeom geom = cache_geom(layout, block_size, Hk, slot);
#define TQ4_STORE_FP8_LAUNCH(L, T)                                                                   \
    launch(&tq4::store::store_fp8_kernel<L, T>, grid, dim3(tq4::kWave * tq4::store::kFp8Waves), st, \
           static_cast<const T *>(key), static_cast<const T *>(value), slot_mapping, kv_cache, rows, Hk,  \
           block_size, cache_block_stride, geom.pos, geom.head)
    switch (dtype * 2 + geom.kl) {
    case TQ4_F32 * 2 + 0: TQ4_STORE_FP8_LAUNCH(0, float); break;
    case TQ4_F32 * 2 + 1: TQ4_STORE_FP8_LAUNCH(1, float); break;
    case TQ4_BF16 * 2 + 0: TQ4_STORE_FP8_LAUNCH(0, __bf16); break;
    case TQ4_BF16 * 2 + 1: TQ4_STORE_FP8_LAUNCH(1, __bf16); break;
    case TQ4_F16 * 2 + 0: TQ4_STORE_FP8_LAUNCH(0, _Float16); break;
    case TQ4_F16 * 2 + 1: TQ4_STORE_FP8_LAUNCH(1, _Float16); break;
    default:
        return fail(TQ4_E_INVALID, "tq4_store_fp8: dtype must be 0 (f32), 1 (bf16) or 2 (f16)");
    }
#undef TQ4_STORE_FP8_LAUNCH
    return launch_status("store_fp8");
}

}  // extern "C"
