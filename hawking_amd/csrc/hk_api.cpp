// hk_api.cpp -- host side of the C ABI (include/hawking_hip.h).
//
// Validates every argument on the host before any launch, owns device
// memory for organs and MoE models, and enqueues kernels on the caller's
// stream.  No entry point falls back to a CPU path.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <cstdlib>
#include <mutex>
#include <string>
#include <vector>

#include "hk_internal.h"
#include "hk_moe.h"
#include "hk_router.h"
#include "hk_synth.h"
#include "hk_tile.h"

using hk::CanonView;

namespace hk {

int set_error(hk_ctx* ctx, int code, const std::string& msg) {
    if (ctx) {
        ctx->last_status = code;
        ctx->last_error = msg;
    }
    return code;
}

int check_hip(hk_ctx* ctx, hipError_t e, const char* what) {
    if (e == hipSuccess) return HK_OK;
    return set_error(ctx, HK_E_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

static inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

static inline bool f16_finite(uint16_t b) { return (b & 0x7C00u) != 0x7C00u; }
// Exact value of a finite f16.
static float f16_to_f32_host(uint16_t h) {
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    const float v = e == 0 ? std::ldexp((float)m, -24) : std::ldexp((float)(m | 0x400u), (int)e - 25);
    return (h & 0x8000u) ? -v : v;
}

static int popcount8(uint8_t v) { return __builtin_popcount(v); }

// Section sizes of one organ in the device layout.
struct Layout {
    size_t scales = 0, codes = 0, tags = 0, row_tab = 0, q2_scales = 0, q2_codes = 0, dense = 0;
    size_t total() const {
        return align256(scales) + align256(codes) + align256(tags) + 2 * align256(row_tab) +
               align256(q2_scales) + align256(q2_codes) + align256(dense);
    }
    size_t packed() const { return scales + codes + tags + q2_scales + q2_codes + dense; }
};

static int validate_shape(hk_ctx* ctx, int kind, int group, uint32_t rows, uint32_t cols) {
    if (rows == 0 || cols == 0) return set_error(ctx, HK_E_GEOMETRY, "organ rows and cols must be positive");
    // the kernels address a tiled organ's sections with 32-bit offsets
    if ((uint64_t)rows * cols > 0xC0000000ull)
        return set_error(ctx, HK_E_GEOMETRY, "organ too large: rows * cols above 3 * 2^30 weights");
    switch (kind) {
    case HK_Q4:
        if (group != 32 && group != 64 && group != 128)
            return set_error(ctx, HK_E_UNSUPPORTED,
                             "uniform Q4 group_size=" + std::to_string(group) + " must be 32, 64 or 128");
        if (cols % (uint32_t)group)
            return set_error(ctx, HK_E_GEOMETRY, "uniform Q4 requires cols to be a multiple of group_size");
        return HK_OK;
    case HK_BIN:
        if (group != 128) return set_error(ctx, HK_E_UNSUPPORTED, "binary organs use group_size 128");
        if (cols % 128)
            return set_error(ctx, HK_E_GEOMETRY,
                             "binary_group kernel requires cols to be a multiple of group_size");
        return HK_OK;
    case HK_MIXED:
        if (cols % 128) return set_error(ctx, HK_E_GEOMETRY, "mixed organs require cols % 128 == 0");
        return HK_OK;
    case HK_Q8:
        if (group != 64) return set_error(ctx, HK_E_UNSUPPORTED, "uniform q8 organs use group_size 64 (HGRAVU01)");
        if (cols % 64) return set_error(ctx, HK_E_GEOMETRY, "uniform q8 organs require cols % 64 == 0");
        return HK_OK;
    case HK_U3:
        if (group != 64) return set_error(ctx, HK_E_UNSUPPORTED, "3-bit factors use group_size 64 (HGRAVS01)");
        if (cols % 32) return set_error(ctx, HK_E_GEOMETRY, "3-bit factors require cols % 32 == 0");
        return HK_OK;
    case HK_F32:
        if (cols % 4) return set_error(ctx, HK_E_GEOMETRY, "dense organs require cols % 4 == 0");
        return HK_OK;
    case HK_BIN_RICE:
        return set_error(ctx, HK_E_UNSUPPORTED, "HGRAVR02 organs are uploaded with hk_organ_upload_rice");
    default:
        return set_error(ctx, HK_E_UNSUPPORTED, "unknown organ kind " + std::to_string(kind));
    }
}

// The GEMV keeps one organ's x image (and a quantization window) in LDS.
static int validate_gemv_cols(hk_ctx* ctx, int kind, uint32_t cols) {
    if (kind == HK_F32 || gemv_lds_bytes(kind, cols) <= GEMV_LDS_LIMIT) return HK_OK;
    uint32_t most = 0;  // the widest organ of this kind whose x image fits
    for (uint32_t c = 32; c <= 65536 && gemv_lds_bytes(kind, c) <= GEMV_LDS_LIMIT; c += 32) most = c;
    return set_error(ctx, HK_E_GEOMETRY, "organ cols=" + std::to_string(cols) +
                                             " exceeds the GEMV's LDS x image (at most " + std::to_string(most) +
                                             " columns for this kind)");
}

static Layout layout_for(int kind, int group, uint32_t rows, uint32_t cols, uint32_t n_bin,
                         uint32_t n_q2) {
    Layout L;
    const size_t n = (size_t)rows * cols;
    switch (kind) {
    case HK_Q4:
        L.scales = n / (size_t)group * 2;
        L.codes = n / 2;
        break;
    case HK_BIN:
        L.scales = n / 128 * 2;
        L.codes = n / 8;
        break;
    case HK_Q8:
        L.scales = n / 64 * 2;
        L.codes = n;
        break;
    case HK_U3:
        L.scales = (n + 63) / 64 * 2;
        L.codes = (n + 63) / 64 * 24;
        break;
    case HK_MIXED: {
        const size_t groups = n / 128;
        L.tags = ((groups + 31) / 32) * 4;
        L.row_tab = ((size_t)rows + 1) * 4;
        L.scales = (size_t)n_bin * 2;
        L.codes = (size_t)n_bin * 16;
        L.q2_scales = (size_t)n_q2 * 4;
        L.q2_codes = (size_t)n_q2 * 32;
        break;
    }
    default:
        L.dense = n * 4;
    }
    return L;
}

// Carves the sections of `L` out of `base` and returns the organ view.
static CanonView place(int kind, int group, uint32_t rows, uint32_t cols, const Layout& L,
                       uint8_t* base) {
    CanonView v{};
    v.kind = kind;
    v.group = group;
    v.rows = rows;
    v.cols = cols;
    uint8_t* p = base;
    v.scales = reinterpret_cast<const uint16_t*>(p);
    p += align256(L.scales);
    v.codes = p;
    p += align256(L.codes);
    v.tags = p;
    p += align256(L.tags);
    v.row_bin = reinterpret_cast<const uint32_t*>(p);
    p += align256(L.row_tab);
    v.row_q2 = reinterpret_cast<const uint32_t*>(p);
    p += align256(L.row_tab);
    v.q2_scales = reinterpret_cast<const uint16_t*>(p);
    p += align256(L.q2_scales);
    v.q2_codes = p;
    p += align256(L.q2_codes);
    v.dense = reinterpret_cast<const float*>(p);
    return v;
}

// Validates the host canonical source of one organ (geometry, finite scales,
// mixed tag counts) and returns its layout.
static int validate_src(hk_ctx* ctx, const hk_organ_src* s, Layout* out) {
    if (!s) return set_error(ctx, HK_E_INVALID_ARG, "organ source is NULL");
    int rc = validate_shape(ctx, s->kind, s->group, s->rows, s->cols);
    if (!rc) rc = validate_gemv_cols(ctx, s->kind, s->cols);
    if (rc) return rc;
    const size_t n = (size_t)s->rows * s->cols;
    if (s->kind == HK_Q4 || s->kind == HK_BIN || s->kind == HK_Q8 || s->kind == HK_U3) {
        if (!s->scales || !s->codes) return set_error(ctx, HK_E_INVALID_ARG, "organ scales/codes are NULL");
        const size_t G = s->kind == HK_Q4 ? s->group : (s->kind == HK_Q8 || s->kind == HK_U3) ? 64 : 128;
        const size_t groups = (n + G - 1) / G;
        for (size_t g = 0; g < groups; ++g)
            if (!f16_finite(s->scales[g]))
                return set_error(ctx, HK_E_NONFINITE, "group " + std::to_string(g) + " scale is not a finite FP16");
    } else if (s->kind == HK_MIXED) {
        if (!s->tags || (s->n_bin && (!s->scales || !s->codes)) || (s->n_q2 && (!s->q2_scales || !s->q2_codes)))
            return set_error(ctx, HK_E_INVALID_ARG, "mixed organ streams are NULL");
        const size_t groups = n / 128;
        size_t nb = 0;
        for (size_t b = 0; b < (groups + 7) / 8; ++b) {
            uint8_t t = s->tags[b];
            if (b == (groups + 7) / 8 - 1 && (groups & 7)) t &= (uint8_t)((1u << (groups & 7)) - 1);
            nb += (size_t)popcount8(t);
        }
        if (nb != s->n_bin || groups - nb != s->n_q2)
            return set_error(ctx, HK_E_GEOMETRY, "mixed tag bitmap disagrees with n_bin / n_q2");
        for (size_t g = 0; g < s->n_bin; ++g)
            if (!f16_finite(s->scales[g])) return set_error(ctx, HK_E_NONFINITE, "mixed binary scale is not finite");
        for (size_t g = 0; g < 2 * (size_t)s->n_q2; ++g)
            if (!f16_finite(s->q2_scales[g])) return set_error(ctx, HK_E_NONFINITE, "mixed Q2 scale is not finite");
    } else {
        if (!s->dense) return set_error(ctx, HK_E_INVALID_ARG, "dense organ data is NULL");
    }
    *out = layout_for(s->kind, s->group, s->rows, s->cols, s->n_bin, s->n_q2);
    return HK_OK;
}

// Copies one validated host organ into device memory at `base` (stream-ordered).
static int copy_src(hk_ctx* ctx, const hk_organ_src* s, const Layout& L, uint8_t* base,
                    CanonView* view, hipStream_t st, std::vector<std::vector<uint32_t>>* keep) {
    CanonView v = place(s->kind, s->group, s->rows, s->cols, L, base);
    auto cp = [&](const void* dst, const void* src, size_t bytes) -> int {
        if (!bytes) return HK_OK;
        return check_hip(ctx, hipMemcpyAsync(const_cast<void*>(dst), src, bytes, hipMemcpyHostToDevice, st),
                         "hipMemcpyAsync (organ upload)");
    };
    int rc = HK_OK;
    if (s->kind == HK_Q4 || s->kind == HK_BIN || s->kind == HK_Q8 || s->kind == HK_U3) {
        if ((rc = cp(v.scales, s->scales, L.scales))) return rc;
        if ((rc = cp(v.codes, s->codes, L.codes))) return rc;
    } else if (s->kind == HK_MIXED) {
        const uint32_t gpr = s->cols / 128;
        std::vector<uint32_t> tags_words(L.tags / 4, 0u);
        std::memcpy(tags_words.data(), s->tags, ((size_t)s->rows * gpr + 7) / 8);
        std::vector<uint32_t> tab(2 * ((size_t)s->rows + 1));
        uint32_t run = 0;
        for (uint32_t r = 0; r <= s->rows; ++r) {
            tab[r] = run;
            tab[s->rows + 1 + r] = r * gpr - run;
            if (r == s->rows) break;
            for (uint32_t g = r * gpr; g < (r + 1) * gpr; ++g) run += (s->tags[g >> 3] >> (g & 7u)) & 1u;
        }
        if ((rc = cp(v.tags, tags_words.data(), L.tags))) return rc;
        if ((rc = cp(v.row_bin, tab.data(), L.row_tab))) return rc;
        if ((rc = cp(v.row_q2, tab.data() + s->rows + 1, L.row_tab))) return rc;
        if ((rc = cp(v.scales, s->scales, L.scales))) return rc;
        if ((rc = cp(v.codes, s->codes, L.codes))) return rc;
        if ((rc = cp(v.q2_scales, s->q2_scales, L.q2_scales))) return rc;
        if ((rc = cp(v.q2_codes, s->q2_codes, L.q2_codes))) return rc;
        // the async copies read host staging vectors: keep them alive until sync
        keep->push_back(std::move(tags_words));
        keep->push_back(std::move(tab));
    } else {
        if ((rc = cp(v.dense, s->dense, L.dense))) return rc;
    }
    *view = v;
    return HK_OK;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---- the no-allocation entry point's workspace
// hk_terminal_greedy_noalloc keeps the head's logits, xn and pick slot in
// this file-scope device array: every device the library runs on holds one
// copy until the process ends.  Host code never passes the array's name to
// a kernel (on the host it is only a stand-in symbol); it uses the device
// address hipGetSymbolAddress returns, looked up once per device on the
// entry point's first call there, with that device current (a context that
// never calls the entry point never looks it up, so it cannot fail on it).
constexpr size_t NOALLOC_LOGITS = (size_t)HK_NOALLOC_HEAD_MAX_ROWS * 4;
constexpr size_t NOALLOC_XN = (size_t)HK_NOALLOC_HEAD_MAX_COLS * 4;
constexpr size_t NOALLOC_BYTES = NOALLOC_LOGITS + NOALLOC_XN + 256;
static __device__ __align__(256) uint8_t scratch[NOALLOC_BYTES];
constexpr int NOALLOC_MAX_DEVICES = 64;
static uint8_t* g_scratch_dev[NOALLOC_MAX_DEVICES] = {};
static std::mutex g_scratch_mu;

// Device address of this device's copy of `scratch`, looked up on the first
// call for the device with that device made current (the caller's current
// device is restored).
static int noalloc_scratch(hk_ctx* ctx, uint8_t** out) {
    if (ctx->device < 0 || ctx->device >= NOALLOC_MAX_DEVICES)
        return set_error(ctx, HK_E_UNSUPPORTED, "no-allocation workspace: device index above 63");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[ctx->device]) {
        int prev = -1;
        hipError_t e = hipGetDevice(&prev);
        if (e != hipSuccess) return check_hip(ctx, e, "hipGetDevice (no-allocation workspace)");
        if (prev != ctx->device && (e = hipSetDevice(ctx->device)) != hipSuccess)
            return check_hip(ctx, e, "hipSetDevice (no-allocation workspace)");
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (prev != ctx->device) (void)hipSetDevice(prev);
        if (e != hipSuccess) return check_hip(ctx, e, "hipGetSymbolAddress (no-allocation workspace)");
        g_scratch_dev[ctx->device] = static_cast<uint8_t*>(ptr);
    }
    *out = g_scratch_dev[ctx->device];
    return HK_OK;
}

}  // namespace hk

using namespace hk;

// ====================================================================== context

extern "C" int hk_ctx_create(int device, hk_ctx** out) {
    if (!out) return HK_E_INVALID_ARG;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return HK_E_HIP;
    if (device < 0 || device >= n) return HK_E_INVALID_ARG;
    if (hipSetDevice(device) != hipSuccess) return HK_E_HIP;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return HK_E_HIP;
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return HK_E_UNSUPPORTED;
    hk_ctx* ctx = new hk_ctx();
    ctx->device = device;
    void* st = nullptr;
    if (hipMalloc(&st, 512) != hipSuccess) {
        delete ctx;
        return HK_E_NOMEM;
    }
    (void)hipMemset(st, 0, 512);
    ctx->dev_status = static_cast<uint32_t*>(st);
    ctx->pack_flag = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(st) + 256);
    *out = ctx;
    return HK_OK;
}

extern "C" void hk_ctx_destroy(hk_ctx* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipDeviceSynchronize();
    if (ctx->dev_status) (void)hipFree(ctx->dev_status);
    delete ctx;
}

extern "C" int hk_stream_control(hk_ctx* ctx, const void* data, size_t nbytes, float* out, uint32_t workgroups,
                                 hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!data || !out || nbytes < 16 || nbytes % 16 || (reinterpret_cast<uintptr_t>(data) & 15u))
        return set_error(ctx, HK_E_INVALID_ARG, "hk_stream_control: need a 16-byte aligned buffer of a multiple of 16 bytes");
    if (workgroups == 0 || workgroups > (1u << 20))
        return set_error(ctx, HK_E_INVALID_ARG, "hk_stream_control: workgroups must be in [1, 2^20]");
    return check_hip(ctx, launch_stream_control(data, nbytes, out, workgroups, static_cast<hipStream_t>(stream)),
                     "stream control launch");
}

extern "C" int hk_last_error(const hk_ctx* ctx, char* buf, size_t len) {
    if (!ctx || !buf || !len) return HK_E_INVALID_ARG;
    std::snprintf(buf, len, "%s", ctx->last_error.c_str());
    return ctx->last_status;
}

extern "C" const char* hk_version(void) { return "hawking-mi355x 0.1 (gfx950)"; }

extern "C" int hk_device_info(hk_ctx* ctx, char* name, size_t len, int* cu_count, size_t* hbm_bytes) {
    if (!ctx) return HK_E_INVALID_ARG;
    hipDeviceProp_t prop;
    int rc = check_hip(ctx, hipGetDeviceProperties(&prop, ctx->device), "hipGetDeviceProperties");
    if (rc) return rc;
    if (name && len) std::snprintf(name, len, "%s (%s)", prop.name, prop.gcnArchName);
    if (cu_count) *cu_count = prop.multiProcessorCount;
    if (hbm_bytes) *hbm_bytes = prop.totalGlobalMem;
    return HK_OK;
}

extern "C" int hk_check_device_status(hk_ctx* ctx, hk_stream stream, uint32_t* bits) {
    if (!ctx || !bits) return HK_E_INVALID_ARG;
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint32_t v = 0;
    int rc = check_hip(ctx, hipMemcpyAsync(&v, ctx->dev_status, 4, hipMemcpyDeviceToHost, st), "status read");
    if (rc) return rc;
    rc = check_hip(ctx, hipStreamSynchronize(st), "hipStreamSynchronize");
    if (rc) return rc;
    *bits = v;
    return check_hip(ctx, hipMemsetAsync(ctx->dev_status, 0, 4, st), "status clear");
}

// ====================================================================== plumbing

extern "C" int hk_malloc(hk_ctx* ctx, size_t bytes, void** out) {
    if (!ctx || !out) return HK_E_INVALID_ARG;
    *out = nullptr;
    if (bytes == 0) bytes = 256;
    if (hipMalloc(out, bytes) != hipSuccess)
        return set_error(ctx, HK_E_NOMEM, "hipMalloc of " + std::to_string(bytes) + " bytes failed");
    return HK_OK;
}

extern "C" int hk_free(hk_ctx* ctx, void* ptr) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!ptr) return HK_OK;
    return check_hip(ctx, hipFree(ptr), "hipFree");
}

static int memcpy_kind(hk_ctx* ctx, void* dst, const void* src, size_t bytes, hk_stream s,
                       hipMemcpyKind kind) {
    if (!ctx || (bytes && (!dst || !src))) return set_error(ctx, HK_E_INVALID_ARG, "memcpy: NULL pointer");
    if (!bytes) return HK_OK;
    return check_hip(ctx, hipMemcpyAsync(dst, src, bytes, kind, static_cast<hipStream_t>(s)), "hipMemcpyAsync");
}

extern "C" int hk_memcpy_htod(hk_ctx* ctx, void* dst, const void* src, size_t bytes, hk_stream s) {
    return memcpy_kind(ctx, dst, src, bytes, s, hipMemcpyHostToDevice);
}
extern "C" int hk_memcpy_dtoh(hk_ctx* ctx, void* dst, const void* src, size_t bytes, hk_stream s) {
    return memcpy_kind(ctx, dst, src, bytes, s, hipMemcpyDeviceToHost);
}
extern "C" int hk_memcpy_dtod(hk_ctx* ctx, void* dst, const void* src, size_t bytes, hk_stream s) {
    return memcpy_kind(ctx, dst, src, bytes, s, hipMemcpyDeviceToDevice);
}

extern "C" int hk_memset(hk_ctx* ctx, void* dst, int value, size_t bytes, hk_stream s) {
    if (!ctx || (bytes && !dst)) return HK_E_INVALID_ARG;
    if (!bytes) return HK_OK;
    return check_hip(ctx, hipMemsetAsync(dst, value, bytes, static_cast<hipStream_t>(s)), "hipMemsetAsync");
}

extern "C" int hk_stream_create(hk_ctx* ctx, hk_stream* out) {
    if (!ctx || !out) return HK_E_INVALID_ARG;
    hipStream_t s;
    int rc = check_hip(ctx, hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    if (rc) return rc;
    *out = s;
    return HK_OK;
}

extern "C" int hk_stream_destroy(hk_ctx* ctx, hk_stream s) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!s) return HK_OK;
    return check_hip(ctx, hipStreamDestroy(static_cast<hipStream_t>(s)), "hipStreamDestroy");
}

extern "C" int hk_stream_synchronize(hk_ctx* ctx, hk_stream s) {
    if (!ctx) return HK_E_INVALID_ARG;
    return check_hip(ctx, hipStreamSynchronize(static_cast<hipStream_t>(s)), "hipStreamSynchronize");
}

extern "C" int hk_device_synchronize(hk_ctx* ctx) {
    if (!ctx) return HK_E_INVALID_ARG;
    return check_hip(ctx, hipDeviceSynchronize(), "hipDeviceSynchronize");
}

extern "C" int hk_event_create(hk_ctx* ctx, void** out) {
    if (!ctx || !out) return HK_E_INVALID_ARG;
    hipEvent_t e;
    int rc = check_hip(ctx, hipEventCreate(&e), "hipEventCreate");
    if (rc) return rc;
    *out = e;
    return HK_OK;
}

extern "C" int hk_event_destroy(hk_ctx* ctx, void* ev) {
    if (!ctx) return HK_E_INVALID_ARG;
    return ev ? check_hip(ctx, hipEventDestroy(static_cast<hipEvent_t>(ev)), "hipEventDestroy") : HK_OK;
}

extern "C" int hk_event_record(hk_ctx* ctx, void* ev, hk_stream s) {
    if (!ctx || !ev) return HK_E_INVALID_ARG;
    return check_hip(ctx, hipEventRecord(static_cast<hipEvent_t>(ev), static_cast<hipStream_t>(s)),
                     "hipEventRecord");
}

extern "C" int hk_event_elapsed_ms(hk_ctx* ctx, void* a, void* b, float* ms) {
    if (!ctx || !a || !b || !ms) return HK_E_INVALID_ARG;
    int rc = check_hip(ctx, hipEventSynchronize(static_cast<hipEvent_t>(b)), "hipEventSynchronize");
    if (rc) return rc;
    return check_hip(ctx, hipEventElapsedTime(ms, static_cast<hipEvent_t>(a), static_cast<hipEvent_t>(b)),
                     "hipEventElapsedTime");
}

// ====================================================================== organs
// Organs are staged in the canonical layout (host upload or device
// generation), then repacked once into the tiled layout the kernels read.

static int repack_into_organ(hk_ctx* ctx, const CanonView& canon, uint32_t n_bin, uint32_t n_q2, hipStream_t st,
                             hk_organ** out) {
    hk_organ* o = new hk_organ();
    o->kind = canon.kind;
    o->alloc_bytes = tiled_bytes(canon.kind, canon.group, canon.rows, canon.cols, n_bin, n_q2, &o->packed_bytes);
    if (hipMalloc(&o->mem, o->alloc_bytes) != hipSuccess) {
        delete o;
        return set_error(ctx, HK_E_NOMEM, "organ allocation failed");
    }
    o->view = tiled_place(canon.kind, canon.group, canon.rows, canon.cols, n_bin, n_q2, static_cast<uint8_t*>(o->mem));
    // the single-organ descriptor; the repack's per-block counts live in a
    // temporary freed after the synchronising upload
    if (hipMalloc(&o->view_dev, align256(sizeof(OrganView))) != hipSuccess) {
        (void)hipFree(o->mem);
        delete o;
        return set_error(ctx, HK_E_NOMEM, "descriptor allocation failed");
    }
    int rc = check_hip(ctx, hipMemcpyAsync(o->view_dev, &o->view, sizeof(OrganView), hipMemcpyHostToDevice, st),
                       "descriptor upload");
    void* counts = nullptr;
    if (!rc && canon.kind == HK_F32) {
        rc = check_hip(ctx, hipMemcpyAsync(const_cast<float*>(o->view.dense), canon.dense,
                                           (size_t)canon.rows * canon.cols * 4, hipMemcpyDeviceToDevice, st),
                       "dense copy");
    } else if (!rc) {
        if (hipMalloc(&counts, 8 * ((size_t)o->view.n_tiles * o->view.steps + 1)) != hipSuccess)
            rc = set_error(ctx, HK_E_NOMEM, "repack count allocation failed");
        else
            rc = check_hip(ctx, launch_repack(canon, o->view, counts, st), "repack launch");
    }
    if (!rc) rc = check_hip(ctx, hipStreamSynchronize(st), "hipStreamSynchronize (repack)");
    if (counts) {
        if (rc) (void)hipStreamSynchronize(st);
        (void)hipFree(counts);
    }
    if (rc) {
        (void)hipFree(o->mem);
        (void)hipFree(o->view_dev);
        delete o;
        return rc;
    }
    *out = o;
    return HK_OK;
}

extern "C" int hk_organ_upload(hk_ctx* ctx, const hk_organ_src* src, hk_stream stream, hk_organ** out) {
    if (!ctx || !out) return HK_E_INVALID_ARG;
    *out = nullptr;
    Layout L;
    int rc = validate_src(ctx, src, &L);
    if (rc) return rc;
    void* stage = nullptr;
    if (hipMalloc(&stage, L.total()) != hipSuccess) return set_error(ctx, HK_E_NOMEM, "staging allocation failed");
    hipStream_t st = static_cast<hipStream_t>(stream);
    std::vector<std::vector<uint32_t>> keep;
    CanonView canon{};
    rc = copy_src(ctx, src, L, static_cast<uint8_t*>(stage), &canon, st, &keep);
    if (!rc) rc = repack_into_organ(ctx, canon, src->n_bin, src->n_q2, st, out);
    (void)hipStreamSynchronize(st);
    (void)hipFree(stage);
    return rc;
}

extern "C" int hk_organ_free(hk_ctx* ctx, hk_organ* o) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!o) return HK_OK;
    int rc = check_hip(ctx, hipFree(o->mem), "hipFree (organ)");
    if (o->view_dev) (void)hipFree(o->view_dev);
    if (o->res_mem) (void)hipFree(o->res_mem);
    delete o;
    return rc;
}

extern "C" int hk_organ_info(const hk_organ* o, int32_t* kind, int32_t* group, uint32_t* rows, uint32_t* cols,
                             size_t* packed_bytes) {
    if (!o) return HK_E_INVALID_ARG;
    if (kind) *kind = o->kind;
    if (group) *group = o->view.group;
    if (rows) *rows = o->view.rows;
    if (cols) *cols = o->view.cols;
    if (packed_bytes) *packed_bytes = o->packed_bytes;
    return HK_OK;
}
static int check_vectors(hk_ctx* ctx, const char* fn, const float* x, size_t x_stride, const float* y,
                         size_t y_stride, uint32_t n, const OrganView& f) {
    if (!x || !y) return set_error(ctx, HK_E_INVALID_ARG, std::string(fn) + ": NULL vector");
    if (!aligned16(x) || !aligned16(y) || (x_stride % 4) || (y_stride % 4))
        return set_error(ctx, HK_E_INVALID_ARG, std::string(fn) + ": x/y must be 16-byte aligned with strides % 4 == 0");
    if (n > 1 && (x_stride < f.cols || y_stride < f.rows))
        return set_error(ctx, HK_E_GEOMETRY, std::string(fn) + ": strides smaller than the organ shape");
    return HK_OK;
}

extern "C" int hk_gemv(hk_ctx* ctx, const hk_organ* o, const float* x, float* y, hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!o) return set_error(ctx, HK_E_INVALID_ARG, "hk_gemv: NULL organ");
    int rc = check_vectors(ctx, "hk_gemv", x, 0, y, 0, 1, o->view);
    if (rc) return rc;
    // the single-organ descriptor was uploaded with the organ
    hipStream_t st = static_cast<hipStream_t>(stream);
    rc = check_hip(ctx, launch_gemv_tiled(static_cast<const OrganView*>(o->view_dev), 1, o->view, x, 0, y, 0, st),
                   "gemv launch");
    if (!rc && o->res_dev)
        rc = check_hip(ctx, launch_rice_apply(o->res_dev, 1, o->view.rows, o->view.cols, o->res_pieces, x, 0, y, 0, st),
                       "rice apply");
    return rc;
}

extern "C" int hk_rice_apply(hk_ctx* ctx, const hk_organ* o, const float* x, float* y, hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!o || !o->res_dev) return set_error(ctx, HK_E_INVALID_ARG, "hk_rice_apply: not an HGRAVR02 organ");
    int rc = check_vectors(ctx, "hk_rice_apply", x, 0, y, 0, 1, o->view);
    if (rc) return rc;
    return check_hip(ctx, launch_rice_apply(o->res_dev, 1, o->view.rows, o->view.cols, o->res_pieces, x, 0, y, 0,
                                            static_cast<hipStream_t>(stream)),
                     "rice apply");
}

extern "C" int hk_gemv_lowrank(hk_ctx* ctx, const hk_organ* left, const hk_organ* right, const float* x, float* mid,
                               float* y, hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!left || !right) return set_error(ctx, HK_E_INVALID_ARG, "hk_gemv_lowrank: NULL factor");
    if (right->view.rows != left->view.cols)
        return set_error(ctx, HK_E_GEOMETRY, "hk_gemv_lowrank: right rows (the rank) must equal left cols");
    int rc = check_vectors(ctx, "hk_gemv_lowrank", x, 0, mid, 0, 1, right->view);
    if (!rc) rc = check_vectors(ctx, "hk_gemv_lowrank", mid, 0, y, 0, 1, left->view);
    if (rc) return rc;
    if (lowrank_fusable(left->view, right->view))
        return check_hip(ctx,
                         launch_lowrank(static_cast<const OrganView*>(left->view_dev),
                                        static_cast<const OrganView*>(right->view_dev), 1, left->view, right->view, x, 0,
                                        mid, 0, y, 0, nullptr, static_cast<hipStream_t>(stream)),
                         "low-rank launch");
    // stream order carries mid from the first launch to the second
    rc = hk_gemv(ctx, right, x, mid, stream);
    return rc ? rc : hk_gemv(ctx, left, mid, y, stream);
}

struct hk_organ_set {
    OrganView* dev = nullptr;
    ResView* res_dev = nullptr;  // HGRAVR02 sets: the residual table
    uint32_t res_pieces = 0;     // the most record pieces of any organ's apply part
    uint32_t res_pieces_256 = 0;  // the same for 256-row parts
    uint32_t res8_pieces = 0, res8_pieces_256 = 0;  // the byte steps' (the fused GEMV's)
    uint32_t n = 0;
    OrganView first{};
};

extern "C" int hk_organ_set_create(hk_ctx* ctx, const hk_organ* const* organs, uint32_t n, hk_organ_set** out) {
    if (!ctx || !out) return HK_E_INVALID_ARG;
    *out = nullptr;
    if (!organs || n == 0) return set_error(ctx, HK_E_INVALID_ARG, "organ set: no organs");
    if (n > 65535) return set_error(ctx, HK_E_INVALID_ARG, "organ set: at most 65535 organs");
    std::vector<OrganView> views(n);
    for (uint32_t i = 0; i < n; ++i) {
        if (!organs[i]) return set_error(ctx, HK_E_INVALID_ARG, "organ set: NULL organ");
        views[i] = organs[i]->view;
        if (views[i].kind != views[0].kind || views[i].rows != views[0].rows || views[i].cols != views[0].cols ||
            views[i].group != views[0].group || organs[i]->kind != organs[0]->kind)
            return set_error(ctx, HK_E_GEOMETRY, "organ set: organs must share kind and shape");
    }
    hk_organ_set* set = new hk_organ_set();
    if (hipMalloc(&set->dev, n * sizeof(OrganView)) != hipSuccess) {
        delete set;
        return set_error(ctx, HK_E_NOMEM, "organ set allocation failed");
    }
    int rc = check_hip(ctx, hipMemcpy(set->dev, views.data(), n * sizeof(OrganView), hipMemcpyHostToDevice),
                       "organ set upload");
    if (rc) {
        (void)hipFree(set->dev);
        delete set;
        return rc;
    }
    if (organs[0]->res_dev) {
        std::vector<ResView> res(n);
        for (uint32_t i = 0; i < n; ++i) {
            res[i] = organs[i]->res;
            set->res_pieces = std::max(set->res_pieces, organs[i]->res_pieces);
            set->res_pieces_256 = std::max(set->res_pieces_256, organs[i]->res_pieces_256);
            set->res8_pieces = std::max(set->res8_pieces, organs[i]->res8_pieces);
            set->res8_pieces_256 = std::max(set->res8_pieces_256, organs[i]->res8_pieces_256);
        }
        if (hipMalloc(&set->res_dev, n * sizeof(ResView)) != hipSuccess) {
            (void)hipFree(set->dev);
            delete set;
            return set_error(ctx, HK_E_NOMEM, "organ set allocation failed");
        }
        rc = check_hip(ctx, hipMemcpy(set->res_dev, res.data(), n * sizeof(ResView), hipMemcpyHostToDevice),
                       "organ set upload");
        if (rc) {
            (void)hipFree(set->dev);
            (void)hipFree(set->res_dev);
            delete set;
            return rc;
        }
    }
    set->n = n;
    set->first = views[0];
    *out = set;
    return HK_OK;
}

extern "C" int hk_organ_set_free(hk_ctx* ctx, hk_organ_set* set) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!set) return HK_OK;
    int rc = check_hip(ctx, hipFree(set->dev), "hipFree (organ set)");
    if (set->res_dev) (void)hipFree(set->res_dev);
    delete set;
    return rc;
}

extern "C" int hk_gemv_set(hk_ctx* ctx, const hk_organ_set* set, const float* x, size_t x_stride, float* y,
                           size_t y_stride, hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!set) return set_error(ctx, HK_E_INVALID_ARG, "hk_gemv_set: NULL set");
    int rc = check_vectors(ctx, "hk_gemv_set", x, x_stride, y, y_stride, set->n, set->first);
    if (rc) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    // HGRAVR02: the residual in the GEMV's epilogue where the launch shape
    // has that form, else the apply after the GEMV
    bool fused = false;
    if (set->res_dev)
        rc = check_hip(ctx,
                       launch_gemv_rice(set->dev, set->res_dev, set->n, set->first, set->res8_pieces_256,
                                        set->res8_pieces, x, x_stride, y, y_stride, st, &fused),
                       "gemv_set launch");
    if (!rc && !fused)
        rc = check_hip(ctx, launch_gemv_tiled(set->dev, set->n, set->first, x, x_stride, y, y_stride, st),
                       "gemv_set launch");
    if (!rc && !fused && set->res_dev)
        rc = check_hip(ctx, launch_rice_apply(set->res_dev, set->n, set->first.rows, set->first.cols, set->res_pieces, x,
                                              x_stride, y, y_stride, st),
                       "rice apply");
    return rc;
}

extern "C" int hk_gemv_lowrank_set(hk_ctx* ctx, const hk_organ_set* left, const hk_organ_set* right, const float* x,
                                   size_t x_stride, float* mid, size_t mid_stride, float* y, size_t y_stride,
                                   hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!left || !right) return set_error(ctx, HK_E_INVALID_ARG, "hk_gemv_lowrank_set: NULL set");
    if (left->n != right->n || right->first.rows != left->first.cols)
        return set_error(ctx, HK_E_GEOMETRY,
                         "hk_gemv_lowrank_set: the sets need as many organs and right rows (the rank) = left cols");
    // x is the right factor's input, y the left factor's output
    OrganView io = right->first;
    io.rows = left->first.rows;
    int rc = check_vectors(ctx, "hk_gemv_lowrank_set", x, x_stride, y, y_stride, left->n, io);
    if (rc) return rc;
    const bool fused = lowrank_fusable(left->first, right->first);
    if (mid) {
        if (!aligned16(mid) || (mid_stride % 4) || (left->n > 1 && mid_stride < right->first.rows))
            return set_error(ctx, HK_E_INVALID_ARG,
                             "hk_gemv_lowrank_set: mid must be 16-byte aligned with mid_stride % 4 == 0 and >= the rank");
    } else if (!fused) {
        return set_error(ctx, HK_E_INVALID_ARG,
                         "hk_gemv_lowrank_set: this shape runs as two launches and needs a mid workspace "
                         "(n x rank floats)");
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (fused)
        return check_hip(ctx,
                         launch_lowrank(left->dev, right->dev, left->n, left->first, right->first, x, x_stride, mid,
                                        mid_stride, y, y_stride, nullptr, st),
                         "low-rank set launch");
    // other shapes: two launches ordered on the stream through the caller's mid
    rc = hk_gemv_set(ctx, right, x, x_stride, mid, mid_stride, stream);
    if (!rc) rc = hk_gemv_set(ctx, left, mid, mid_stride, y, y_stride, stream);
    return rc;
}

extern "C" int hk_gemv_batch(hk_ctx* ctx, const hk_organ* const* organs, uint32_t n, const float* x,
                             size_t x_stride, float* y, size_t y_stride, hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    hk_organ_set* set = nullptr;
    int rc = hk_organ_set_create(ctx, organs, n, &set);
    if (rc) return rc;
    rc = hk_gemv_set(ctx, set, x, x_stride, y, y_stride, stream);
    if (!rc) rc = check_hip(ctx, hipStreamSynchronize(static_cast<hipStream_t>(stream)), "hipStreamSynchronize");
    int rc2 = hk_organ_set_free(ctx, set);
    return rc ? rc : rc2;
}

static int upload_rice(hk_ctx* ctx, const hk_rice_q1* s, hipStream_t st, hk_organ** out);

// Synthetic HGRAVR02 organ: weights from the generator, the device packer at
// the shipped 2% outlier ratio, then the ordinary upload.
static int synthetic_rice(hk_ctx* ctx, uint32_t rows, uint32_t cols, uint64_t key, float sigma, hipStream_t st,
                          hk_organ** out) {
    if (rows == 0 || cols == 0 || cols % 128 || (uint64_t)rows * cols > 0x7FFFFFFFull)
        return set_error(ctx, HK_E_GEOMETRY, "synthetic HGRAVR02 organs need cols % 128 == 0 and rows * cols < 2^31");
    const size_t n = (size_t)rows * cols, count = (size_t)std::ceil((double)n * 0.02);
    const size_t a_w = align256(n * 4), a_s = align256(n / 128 * 2), a_g = align256(n / 8),
                 a_r = align256((count + 7) / 8), cap = align256(n / 8 + 17 * count / 8 + 64);
    uint8_t* m = nullptr;
    if (hipMalloc(&m, a_w + a_s + a_g + a_r + cap) != hipSuccess)
        return set_error(ctx, HK_E_NOMEM, "synthetic staging allocation failed");
    float* w = reinterpret_cast<float*>(m);
    hk_rice_q1 src{};
    int rc = check_hip(ctx, launch_synth_normal(key, 0, n, sigma, w, st), "synth launch");
    if (!rc)
        rc = hk_pack_binary_rice(ctx, w, rows, cols, 0.02, reinterpret_cast<uint16_t*>(m + a_w), m + a_w + a_s,
                                 m + a_w + a_s + a_g, m + a_w + a_s + a_g + a_r, cap, &src, st);
    if (!rc) rc = upload_rice(ctx, &src, st, out);
    (void)hipStreamSynchronize(st);
    (void)hipFree(m);
    return rc;
}

extern "C" int hk_organ_synthetic(hk_ctx* ctx, int32_t kind, int32_t group, uint32_t rows, uint32_t cols, uint64_t key,
                                  uint64_t coin_key, float sigma, hk_stream stream, hk_organ** out) {
    if (!ctx || !out) return HK_E_INVALID_ARG;
    *out = nullptr;
    if (kind == HK_BIN_RICE) {
        int rc = validate_gemv_cols(ctx, HK_BIN, cols);
        return rc ? rc : synthetic_rice(ctx, rows, cols, key, sigma, static_cast<hipStream_t>(stream), out);
    }
    if (kind == HK_BIN || kind == HK_MIXED) group = 128;
    if (kind == HK_Q8 || kind == HK_U3) group = 64;
    int rc = validate_shape(ctx, kind, group, rows, cols);
    if (!rc) rc = validate_gemv_cols(ctx, kind, cols);
    if (rc) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    void* tmp = nullptr;
    if (hipMalloc(&tmp, sizeof(SynthJob) + 256) != hipSuccess) return set_error(ctx, HK_E_NOMEM, "job allocation failed");
    SynthJob* jd = static_cast<SynthJob*>(tmp);
    uint32_t* aux = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(tmp) + sizeof(SynthJob) + 64);
    SynthJob j{};
    j.key = key;
    j.coin_key = coin_key;
    j.sigma = sigma;
    j.group = group;
    j.rows = rows;
    j.cols = cols;
    const size_t G = kind == HK_F32 ? 128 : (size_t)group;
    const size_t groups = ((size_t)rows * cols + G - 1) / G;
    uint32_t nbin = 0;
    rc = check_hip(ctx, hipMemsetAsync(aux, 0, 8, st), "memset");
    if (!rc && kind == HK_MIXED) {
        rc = check_hip(ctx, hipMemcpyAsync(jd, &j, sizeof(j), hipMemcpyHostToDevice, st), "job upload");
        if (!rc) rc = check_hip(ctx, launch_synth_mixed_count(jd, 1, groups, aux + 1, st), "count");
        if (!rc) rc = check_hip(ctx, hipMemcpyAsync(&nbin, aux + 1, 4, hipMemcpyDeviceToHost, st), "count read");
        if (!rc) rc = check_hip(ctx, hipStreamSynchronize(st), "sync");
    }
    const uint32_t nq2 = kind == HK_MIXED ? (uint32_t)(groups - nbin) : 0;
    void* stage = nullptr;
    CanonView canon{};
    if (!rc) {
        const Layout L = layout_for(kind, group, rows, cols, nbin, nq2);
        if (hipMalloc(&stage, L.total()) != hipSuccess) {
            rc = set_error(ctx, HK_E_NOMEM, "staging allocation failed");
        } else {
            canon = place(kind, group, rows, cols, L, static_cast<uint8_t*>(stage));
            j.scales = const_cast<uint16_t*>(canon.scales);
            j.codes = const_cast<uint8_t*>(canon.codes);
            j.tags = const_cast<uint8_t*>(canon.tags);
            j.q2_scales = const_cast<uint16_t*>(canon.q2_scales);
            j.q2_codes = const_cast<uint8_t*>(canon.q2_codes);
            j.row_bin = const_cast<uint32_t*>(canon.row_bin);
            j.row_q2 = const_cast<uint32_t*>(canon.row_q2);
            j.dense = const_cast<float*>(canon.dense);
            rc = check_hip(ctx, hipMemcpyAsync(jd, &j, sizeof(j), hipMemcpyHostToDevice, st), "job upload");
            if (!rc) rc = check_hip(ctx, launch_synth_jobs(kind, jd, 1, groups, aux, st), "synth organ");
            uint32_t bad = 0;
            if (!rc) rc = check_hip(ctx, hipMemcpyAsync(&bad, aux, 4, hipMemcpyDeviceToHost, st), "flag read");
            if (!rc) rc = check_hip(ctx, hipStreamSynchronize(st), "sync");
            if (!rc && bad) rc = set_error(ctx, HK_E_NONFINITE, "synthetic organ has a non-finite scale");
        }
    }
    if (!rc) rc = repack_into_organ(ctx, canon, nbin, nq2, st, out);
    (void)hipStreamSynchronize(st);
    if (stage) (void)hipFree(stage);
    (void)hipFree(tmp);
    return rc;
}

// Rice expand into the CSR the apply reads (unpack_rice + expand_rice_indices +
// rice_q1_row_ptr, q80_mixed_decode.rs:348-381,462-507), on the host at bind
// time as the reference's parse does; records are column << 1 | sign.  Each
// row's records are then padded to a multiple of 4 with cols << 1 (the apply
// reads a row four records at a time and the padding adds -0, which changes
// no sum), and recs to a multiple of 8 (16-byte pieces).  Returns "" or the
// error.
static std::string rice_expand_csr(const uint8_t* rice, size_t len, uint32_t first, uint32_t k, size_t count,
                                   uint32_t rows, uint32_t cols, const uint8_t* signs, std::vector<uint32_t>& row_ptr,
                                   std::vector<uint16_t>& recs) {
    const uint64_t limit = (uint64_t)rows * cols;
    row_ptr.assign((size_t)rows + 1, 0u);
    recs.assign((count + 7) & ~(size_t)7, 0u);
    auto put = [&](size_t i, uint64_t f) {
        recs[i] = (uint16_t)(((f % cols) << 1) | ((uint32_t)(signs[i >> 3] >> (i & 7u)) & 1u));
        row_ptr[f / cols + 1] += 1;
    };
    if (first >= limit) return "rice residual index out of range";
    put(0, first);
    uint64_t pos = 0, acc = first;
    const uint64_t end = (uint64_t)len * 8u;
    for (size_t i = 1; i < count; ++i) {
        uint64_t q = 0;
        for (;;) {
            if (pos >= end) return "rice stream overran its payload";
            const uint32_t b = (rice[pos >> 3] >> (pos & 7u)) & 1u;
            ++pos;
            if (!b) break;
            if (++q > 0xFFFFFFFFull) return "rice quotient overflow";
        }
        uint32_t rem = 0;
        for (uint32_t b = 0; b < k; ++b, ++pos) {
            if (pos >= end) return "rice stream overran its payload";
            rem |= (uint32_t)((rice[pos >> 3] >> (pos & 7u)) & 1u) << b;
        }
        acc += (uint64_t)((uint32_t)(q << k) | rem);
        if (acc > 0xFFFFFFFFull) return "rice index exceeds u32";
        if (acc >= limit) return "rice residual index out of range";
        put(i, acc);
    }
    for (uint32_t r = 0; r < rows; ++r) row_ptr[r + 1] += row_ptr[r];
    std::vector<uint32_t> pp((size_t)rows + 1, 0u);
    for (uint32_t r = 0; r < rows; ++r) pp[r + 1] = pp[r] + ((row_ptr[r + 1] - row_ptr[r] + 3u) & ~3u);
    std::vector<uint16_t> pr(((size_t)pp[rows] + 7) & ~(size_t)7, (uint16_t)(cols << 1));
    for (uint32_t r = 0; r < rows; ++r)
        std::copy(recs.begin() + row_ptr[r], recs.begin() + row_ptr[r + 1], pr.begin() + pp[r]);
    row_ptr.swap(pp);
    recs.swap(pr);
    return "";
}

// The fused GEMV's byte steps (ResView) from the padded CSR: each real
// record of a row (its padding, column cols, ends it) at table index
// 3 col + sign, reached from the previous index (-1 at the row's start) in
// steps of at most 255 through -0 entries (3c + 2); the row padded to 4 bytes
// with steps onto the next -0 entries (at most 3 + 3 + 3 past the last real
// index 3 cols - 2, inside the table's 3 cols + 8 entries); the stream padded
// to 16 bytes.
static void rice_step_records(const std::vector<uint32_t>& row_ptr, const std::vector<uint16_t>& recs, uint32_t rows,
                              uint32_t cols, std::vector<uint32_t>& rp8, std::vector<uint8_t>& r8) {
    rp8.assign((size_t)rows + 1, 0u);
    r8.clear();
    for (uint32_t r = 0; r < rows; ++r) {
        int64_t v = -1;
        const size_t start = r8.size();
        for (uint32_t k = row_ptr[r]; k < row_ptr[r + 1]; ++k) {
            const uint32_t u = recs[k];
            if ((u >> 1) >= cols) break;
            const int64_t t = 3 * (int64_t)(u >> 1) + (int64_t)(u & 1u);
            while (t - v > 255) {
                const int64_t z = v + 255 - (v + 253) % 3;  // the farthest -0 entry in reach (v + 253 >= 252)
                r8.push_back((uint8_t)(z - v));
                v = z;
            }
            r8.push_back((uint8_t)(t - v));
            v = t;
        }
        while ((r8.size() - start) % 4u) {
            const int64_t z = v + 1 + (3 - (v + 1 + 1) % 3) % 3;  // the nearest -0 entry past v (v + 2 >= 1)
            r8.push_back((uint8_t)(z - v));
            v = z;
        }
        rp8[r + 1] = (uint32_t)r8.size();
    }
    r8.resize((r8.size() + 15u) & ~(size_t)15, 0u);
}

// Bind of an HGRAVR02 body: base repack on the device, Rice expand + CSR.
static int upload_rice(hk_ctx* ctx, const hk_rice_q1* s, hipStream_t st, hk_organ** out) {
    const size_t n = (size_t)s->rows * s->cols, count = s->outlier_count;
    const size_t sign_bytes = (count + 7) / 8;
    // the stream and signs on the host (the pointers may be device memory)
    std::vector<uint8_t> rice(s->rice_bytes), signs(sign_bytes);
    int rc = HK_OK;
    if (s->rice_bytes)
        rc = check_hip(ctx, hipMemcpy(rice.data(), s->rice, s->rice_bytes, hipMemcpyDefault), "rice stream read");
    if (!rc) rc = check_hip(ctx, hipMemcpy(signs.data(), s->residual_signs, sign_bytes, hipMemcpyDefault), "sign read");
    if (rc) return rc;
    std::vector<uint32_t> row_ptr;
    std::vector<uint16_t> recs;
    const std::string err = rice_expand_csr(rice.data(), rice.size(), s->first_index, s->rice_k, count, s->rows, s->cols,
                                            signs.data(), row_ptr, recs);
    if (!err.empty()) return set_error(ctx, HK_E_GEOMETRY, err);
    std::vector<uint32_t> rp8;
    std::vector<uint8_t> r8;
    rice_step_records(row_ptr, recs, s->rows, s->cols, rp8, r8);

    const Layout L = layout_for(HK_BIN, 128, s->rows, s->cols, 0, 0);
    uint8_t* stage = nullptr;
    if (hipMalloc(&stage, L.total() + 256) != hipSuccess) return set_error(ctx, HK_E_NOMEM, "staging allocation failed");
    CanonView canon = place(HK_BIN, 128, s->rows, s->cols, L, stage);
    uint32_t* status = reinterpret_cast<uint32_t*>(stage + L.total());
    uint32_t hst = 0;
    rc = check_hip(ctx, hipMemsetAsync(status, 0, 4, st), "hipMemsetAsync");
    if (!rc)
        rc = check_hip(ctx, hipMemcpyAsync(const_cast<uint16_t*>(canon.scales), s->bin_scales, L.scales, hipMemcpyDefault, st),
                       "hipMemcpyAsync (HGRAVR02 upload)");
    if (!rc)
        rc = check_hip(ctx, hipMemcpyAsync(const_cast<uint8_t*>(canon.codes), s->bin_signs, L.codes, hipMemcpyDefault, st),
                       "hipMemcpyAsync (HGRAVR02 upload)");
    if (!rc) rc = check_hip(ctx, launch_f16_check(canon.scales, n / 128, status, st), "scale check");
    if (!rc) rc = check_hip(ctx, hipMemcpyAsync(&hst, status, 4, hipMemcpyDeviceToHost, st), "status read");
    if (!rc) rc = check_hip(ctx, hipStreamSynchronize(st), "hipStreamSynchronize (HGRAVR02 upload)");
    if (!rc && hst) rc = set_error(ctx, HK_E_NONFINITE, "HGRAVR02 binary scale is not a finite FP16");
    hk_organ* o = nullptr;
    if (!rc) rc = repack_into_organ(ctx, canon, 0, 0, st, &o);
    if (!rc) {
        const size_t a_rp = align256(row_ptr.size() * 4), a_rec = align256(recs.size() * 2);
        const size_t a_rp8 = align256(rp8.size() * 4), a_r8 = align256(r8.size());
        if (hipMalloc(&o->res_mem, a_rp + a_rec + a_rp8 + a_r8 + sizeof(ResView)) != hipSuccess) {
            rc = set_error(ctx, HK_E_NOMEM, "residual allocation failed");
        } else {
            uint8_t* m = static_cast<uint8_t*>(o->res_mem);
            o->res.row_ptr = reinterpret_cast<const uint32_t*>(m);
            o->res.recs = reinterpret_cast<const uint16_t*>(m + a_rp);
            o->res.rows = s->rows;
            o->res.cols = s->cols;
            o->res.scale = f16_to_f32_host(s->residual_scale_f16);
            o->res.count = row_ptr[s->rows];
            o->res.row_ptr8 = reinterpret_cast<const uint32_t*>(m + a_rp + a_rec);
            o->res.recs8 = m + a_rp + a_rec + a_rp8;
            o->res.count8 = rp8[s->rows];
            o->res_pieces = rice_part_pieces(row_ptr.data(), s->rows, RICE_APPLY_ROWS);
            o->res_pieces_256 = rice_part_pieces(row_ptr.data(), s->rows, 256u);
            o->res8_pieces = rice_part_pieces8(rp8.data(), s->rows, 512u);
            o->res8_pieces_256 = rice_part_pieces8(rp8.data(), s->rows, 256u);
            ResView* rd = reinterpret_cast<ResView*>(m + a_rp + a_rec + a_rp8 + a_r8);
            rc = check_hip(ctx, hipMemcpy(m, row_ptr.data(), row_ptr.size() * 4, hipMemcpyHostToDevice), "row_ptr upload");
            if (!rc) rc = check_hip(ctx, hipMemcpy(m + a_rp, recs.data(), recs.size() * 2, hipMemcpyHostToDevice), "record upload");
            if (!rc)
                rc = check_hip(ctx, hipMemcpy(m + a_rp + a_rec, rp8.data(), rp8.size() * 4, hipMemcpyHostToDevice),
                               "step row_ptr upload");
            if (!rc)
                rc = check_hip(ctx, hipMemcpy(m + a_rp + a_rec + a_rp8, r8.data(), r8.size(), hipMemcpyHostToDevice),
                               "step record upload");
            if (!rc) rc = check_hip(ctx, hipMemcpy(rd, &o->res, sizeof(ResView), hipMemcpyHostToDevice), "residual upload");
            o->res_dev = rd;
        }
        o->kind = HK_BIN_RICE;
        o->packed_bytes = n / 8 + n / 128 * 2 + 4 + s->rice_bytes + 2 + sign_bytes;
        if (rc) {
            (void)hk_organ_free(ctx, o);
            o = nullptr;
        }
    }
    (void)hipStreamSynchronize(st);
    (void)hipFree(stage);
    if (!rc) *out = o;
    return rc;
}

extern "C" int hk_organ_upload_rice(hk_ctx* ctx, const hk_rice_q1* s, hk_stream stream, hk_organ** out) {
    if (!ctx || !out) return HK_E_INVALID_ARG;
    *out = nullptr;
    if (!s) return set_error(ctx, HK_E_INVALID_ARG, "hk_organ_upload_rice: NULL source");
    if (s->rows == 0 || s->cols == 0 || s->cols % 128)
        return set_error(ctx, HK_E_GEOMETRY, "HGRAVR02 organs require rows > 0 and cols % 128 == 0");
    if (s->cols >= 32768) return set_error(ctx, HK_E_GEOMETRY, "HGRAVR02 organs require cols < 32768");
    if ((uint64_t)s->rows * s->cols > 0xFFFFFFFFull)
        return set_error(ctx, HK_E_GEOMETRY, "HGRAVR02 flat indices are u32: rows * cols too large");
    int rc = validate_gemv_cols(ctx, HK_BIN, s->cols);
    if (rc) return rc;
    if (s->outlier_count == 0) return set_error(ctx, HK_E_GEOMETRY, "rice residual requires at least one outlier");
    if (s->outlier_count > (size_t)s->rows * s->cols)
        return set_error(ctx, HK_E_GEOMETRY, "outlier_count exceeds rows * cols");
    if (s->rice_k > 31) return set_error(ctx, HK_E_GEOMETRY, "rice_k must be below 32");
    if (!s->bin_scales || !s->bin_signs || !s->residual_signs || (s->outlier_count > 1 && s->rice_bytes && !s->rice))
        return set_error(ctx, HK_E_INVALID_ARG, "HGRAVR02 streams are NULL");
    if ((s->residual_scale_f16 & 0x7C00u) == 0x7C00u)
        return set_error(ctx, HK_E_NONFINITE, "HGRAVR02 residual scale is not a finite FP16");
    return upload_rice(ctx, s, static_cast<hipStream_t>(stream), out);
}

extern "C" int hk_decode_rows(hk_ctx* ctx, const hk_organ* o, uint32_t row0, uint32_t nrows, float* out,
                              hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!o || !out) return set_error(ctx, HK_E_INVALID_ARG, "hk_decode_rows: NULL argument");
    if ((uint64_t)row0 + nrows > o->view.rows) return set_error(ctx, HK_E_GEOMETRY, "hk_decode_rows: rows out of range");
    hipStream_t st = static_cast<hipStream_t>(stream);
    int rc = check_hip(ctx, launch_decode_rows(o->view, row0, nrows, out, st), "decode launch");
    if (!rc && o->res_dev) rc = check_hip(ctx, launch_rice_decode_add(o->res, row0, nrows, out, st), "rice decode");
    return rc;
}

// ====================================================================== packers / generator

static int finish_pack(hk_ctx* ctx, hipStream_t st, uint32_t* bad_dev, hipError_t launch) {
    int rc = check_hip(ctx, launch, "pack launch");
    if (rc) return rc;
    uint32_t bad = 0;
    rc = check_hip(ctx, hipMemcpyAsync(&bad, bad_dev, 4, hipMemcpyDeviceToHost, st), "pack status read");
    if (!rc) rc = check_hip(ctx, hipStreamSynchronize(st), "hipStreamSynchronize (pack)");
    if (rc) return rc;
    if (bad) return set_error(ctx, HK_E_NONFINITE, "source tensor contains a non-finite value or scale");
    return HK_OK;
}

static int pack_prologue(hk_ctx* ctx, hipStream_t st, uint32_t** bad) {
    *bad = ctx->pack_flag;
    return check_hip(ctx, hipMemsetAsync(ctx->pack_flag, 0, 4, st), "hipMemsetAsync (pack flag)");
}

extern "C" int hk_pack_q4(hk_ctx* ctx, const float* w, uint32_t rows, uint32_t cols, int32_t group,
                          uint16_t* scales, uint8_t* codes, hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    int rc = validate_shape(ctx, HK_Q4, group, rows, cols);
    if (rc) return rc;
    if (!w || !scales || !codes || !aligned16(codes) || !aligned16(w))
        return set_error(ctx, HK_E_INVALID_ARG, "hk_pack_q4: NULL or misaligned pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint32_t* bad;
    if ((rc = pack_prologue(ctx, st, &bad))) return rc;
    const size_t groups = (size_t)rows * cols / (size_t)group;
    return finish_pack(ctx, st, bad, launch_pack_q4(w, groups, group, scales, codes, bad, st));
}

extern "C" int hk_pack_bin(hk_ctx* ctx, const float* w, uint32_t rows, uint32_t cols, uint16_t* scales,
                           uint8_t* signs, hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    int rc = validate_shape(ctx, HK_BIN, 128, rows, cols);
    if (rc) return rc;
    if (!w || !scales || !signs || !aligned16(signs))
        return set_error(ctx, HK_E_INVALID_ARG, "hk_pack_bin: NULL or misaligned pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint32_t* bad;
    if ((rc = pack_prologue(ctx, st, &bad))) return rc;
    return finish_pack(ctx, st, bad, launch_pack_bin(w, (size_t)rows * cols / 128, scales, signs, bad, st));
}

extern "C" int hk_pack_q8(hk_ctx* ctx, const float* w, uint32_t rows, uint32_t cols, uint16_t* scales,
                          uint8_t* codes, hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    int rc = validate_shape(ctx, HK_Q8, 64, rows, cols);
    if (rc) return rc;
    if (!w || !scales || !codes || !aligned16(codes))
        return set_error(ctx, HK_E_INVALID_ARG, "hk_pack_q8: NULL or misaligned pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint32_t* bad;
    if ((rc = pack_prologue(ctx, st, &bad))) return rc;
    return finish_pack(ctx, st, bad, launch_pack_q8(w, (size_t)rows * cols / 64, scales, codes, bad, st));
}

extern "C" int hk_pack_u3(hk_ctx* ctx, const float* w, size_t count, uint16_t* scales, uint8_t* codes,
                          hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (count == 0) return set_error(ctx, HK_E_GEOMETRY, "hk_pack_u3: count must be positive");
    if (!w || !scales || !codes || !aligned16(codes))
        return set_error(ctx, HK_E_INVALID_ARG, "hk_pack_u3: NULL or misaligned pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint32_t* bad;
    int rc;
    if ((rc = pack_prologue(ctx, st, &bad))) return rc;
    return finish_pack(ctx, st, bad, launch_pack_u3(w, count, scales, codes, bad, st));
}

extern "C" int hk_pack_binary_rice(hk_ctx* ctx, const float* w, uint32_t rows, uint32_t cols, double ratio,
                                   uint16_t* bin_scales, uint8_t* bin_signs, uint8_t* residual_signs, uint8_t* rice,
                                   size_t rice_cap, hk_rice_q1* out, hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!out) return set_error(ctx, HK_E_INVALID_ARG, "hk_pack_binary_rice: NULL out");
    if (rows == 0 || cols == 0 || cols % 128)
        return set_error(ctx, HK_E_GEOMETRY, "hk_pack_binary_rice: rows > 0 and cols % 128 == 0 required");
    if ((uint64_t)rows * cols > 0x7FFFFFFFull)
        return set_error(ctx, HK_E_GEOMETRY, "hk_pack_binary_rice: rows * cols must stay below 2^31");
    if (!(ratio > 0.0 && ratio <= 0.1))
        return set_error(ctx, HK_E_INVALID_ARG, "rice_q1 outlier ratio must be in (0, 0.1]");
    if (!w || !bin_scales || !bin_signs || !residual_signs || !rice || !aligned16(rice) || !aligned16(w))
        return set_error(ctx, HK_E_INVALID_ARG, "hk_pack_binary_rice: NULL or misaligned pointer");
    RicePackResult r{};
    const hipError_t e = pack_binary_rice_device(w, rows, cols, ratio, bin_scales, bin_signs, residual_signs, rice,
                                                 rice_cap, &r, static_cast<hipStream_t>(stream));
    *out = hk_rice_q1{};
    out->rows = rows;
    out->cols = cols;
    out->bin_scales = bin_scales;
    out->bin_signs = bin_signs;
    out->first_index = r.first;
    out->rice_k = r.k;
    out->rice = r.count > 1 ? rice : nullptr;
    out->rice_bytes = r.rice_bytes;
    out->outlier_count = r.count;
    out->residual_scale_f16 = r.scale;
    out->residual_signs = residual_signs;
    if (e == hipErrorInvalidValue && r.rice_bytes)
        return set_error(ctx, HK_E_INVALID_ARG, "hk_pack_binary_rice: rice_cap below the " +
                                                    std::to_string(((r.rice_bytes + 3) / 4) * 4) + " bytes needed");
    int rc = check_hip(ctx, e, "pack_binary_rice");
    if (rc) return rc;
    if (r.bad) return set_error(ctx, HK_E_NONFINITE, "source tensor contains a non-finite value or scale");
    return HK_OK;
}

extern "C" int hk_pack_q2(hk_ctx* ctx, const float* w, size_t count, uint16_t* scales, uint8_t* codes,
                          hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (count == 0 || count % 64) return set_error(ctx, HK_E_GEOMETRY, "hk_pack_q2: count must be a positive multiple of 64");
    if (!w || !scales || !codes || !aligned16(codes))
        return set_error(ctx, HK_E_INVALID_ARG, "hk_pack_q2: NULL or misaligned pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint32_t* bad;
    int rc;
    if ((rc = pack_prologue(ctx, st, &bad))) return rc;
    return finish_pack(ctx, st, bad, launch_pack_q2(w, count / 64, scales, codes, bad, st));
}

extern "C" int hk_pack_mixed(hk_ctx* ctx, const float* w, uint32_t rows, uint32_t cols, const uint8_t* is_binary,
                             uint8_t* tags, uint16_t* bin_scales, uint8_t* bin_signs, uint32_t bin_cap,
                             uint16_t* q2_scales, uint8_t* q2_codes, uint32_t q2_cap, uint32_t* n_bin_out,
                             hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    int rc = validate_shape(ctx, HK_MIXED, 128, rows, cols);
    if (rc) return rc;
    if (!w || !is_binary || !tags || !n_bin_out || !aligned16(w))
        return set_error(ctx, HK_E_INVALID_ARG, "hk_pack_mixed: NULL or misaligned pointer");
    if ((bin_cap && (!bin_scales || !bin_signs || !aligned16(bin_signs))) ||
        (q2_cap && (!q2_scales || !q2_codes || !aligned16(q2_codes))) ||
        (reinterpret_cast<uintptr_t>(bin_scales) & 1u) || (reinterpret_cast<uintptr_t>(q2_scales) & 1u))
        return set_error(ctx, HK_E_INVALID_ARG, "hk_pack_mixed: NULL or misaligned output section");
    const size_t groups = (size_t)rows * cols / 128;
    if (groups > 0xFFFFFFFFull) return set_error(ctx, HK_E_GEOMETRY, "hk_pack_mixed: more than 2^32 groups");
    hipStream_t st = static_cast<hipStream_t>(stream);
    // pass 1: tags and the binary count (into the packer flag's neighbour word)
    uint32_t* bad;
    if ((rc = pack_prologue(ctx, st, &bad))) return rc;
    uint32_t* count = ctx->pack_flag + 1;
    uint32_t nb = 0;
    rc = check_hip(ctx, hipMemsetAsync(count, 0, 4, st), "hipMemsetAsync (mixed count)");
    if (!rc) rc = check_hip(ctx, launch_mixed_tags_from_sel(is_binary, groups, tags, count, st), "mixed tags");
    if (!rc) rc = check_hip(ctx, hipMemcpyAsync(&nb, count, 4, hipMemcpyDeviceToHost, st), "mixed count read");
    if (!rc) rc = check_hip(ctx, hipStreamSynchronize(st), "hipStreamSynchronize (mixed count)");
    if (rc) return rc;
    *n_bin_out = nb;
    const uint32_t nq = (uint32_t)(groups - nb);
    if (nb > bin_cap || nq > q2_cap)
        return set_error(ctx, HK_E_INVALID_ARG, "hk_pack_mixed: the selector has " + std::to_string(nb) +
                                                    " binary and " + std::to_string(nq) +
                                                    " Q2 groups, above bin_cap / q2_cap");
    // passes 2-3: per-row prefix tables (temporary), then one thread per group
    void* tmp = nullptr;
    if (hipMalloc(&tmp, align256(sizeof(SynthJob)) + 2 * align256(((size_t)rows + 1) * 4)) != hipSuccess)
        return set_error(ctx, HK_E_NOMEM, "hk_pack_mixed: row table allocation failed");
    uint8_t* tp = static_cast<uint8_t*>(tmp);
    SynthJob j{};
    j.group = 128;
    j.rows = rows;
    j.cols = cols;
    j.scales = bin_scales;
    j.codes = bin_signs;
    j.tags = tags;
    j.q2_scales = q2_scales;
    j.q2_codes = q2_codes;
    j.row_bin = reinterpret_cast<uint32_t*>(tp + align256(sizeof(SynthJob)));
    j.row_q2 = reinterpret_cast<uint32_t*>(tp + align256(sizeof(SynthJob)) + align256(((size_t)rows + 1) * 4));
    j.w = w;
    rc = check_hip(ctx, hipMemcpyAsync(tmp, &j, sizeof(j), hipMemcpyHostToDevice, st), "mixed job upload");
    if (!rc) rc = finish_pack(ctx, st, bad, launch_mixed_pack_buffer(static_cast<SynthJob*>(tmp), groups, bad, st));
    (void)hipStreamSynchronize(st);
    (void)hipFree(tmp);
    return rc;
}

extern "C" uint64_t hk_stream_key(uint64_t seed, uint64_t stream_id) { return hk::stream_key(seed, stream_id); }

extern "C" int hk_synth_normal(hk_ctx* ctx, uint64_t key, uint64_t first, size_t count, float sigma, float* out,
                               hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!out) return set_error(ctx, HK_E_INVALID_ARG, "hk_synth_normal: NULL output");
    if (!count) return HK_OK;
    return check_hip(ctx, launch_synth_normal(key, first, count, sigma, out, static_cast<hipStream_t>(stream)),
                     "synth launch");
}

// ====================================================================== terminal head

// The head's launches: fused for a q8 lm_head the fused GEMV takes, else norm,
// GEMV and pick.  `pick` holds 16 zero bytes and is left zeroed.
static int head_greedy(hk_ctx* ctx, const float* hidden, const float* norm_w, float eps, const hk_organ* lm_head,
                       uint32_t n_valid, float* xn, float* logits, uint64_t* pick, int32_t* token, hipStream_t st) {
    if (head_gemv_fusable(lm_head->view) && aligned16(norm_w) && aligned16(xn))
        return check_hip(ctx,
                         launch_head_fused(static_cast<const OrganView*>(lm_head->view_dev), lm_head->view, hidden,
                                           norm_w, eps, xn, logits, n_valid, pick, token, ctx->dev_status, st),
                         "terminal head");
    int rc = check_hip(ctx, launch_head_norm(hidden, norm_w, lm_head->view.cols, eps, xn, token, pick,
                                             ctx->dev_status, st),
                       "head norm");
    if (!rc) rc = hk_gemv(ctx, lm_head, xn, logits, st);
    if (!rc) rc = check_hip(ctx, launch_head_argmax(logits, n_valid, pick, token, ctx->dev_status, st), "head argmax");
    return rc;
}

extern "C" int hk_terminal_greedy(hk_ctx* ctx, const float* hidden, const float* norm_w, float eps,
                                  const hk_organ* lm_head, uint32_t n_valid, float* xn, float* logits, uint64_t* pick,
                                  int32_t* token, hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!lm_head || !hidden || !norm_w || !xn || !logits || !pick || !token)
        return set_error(ctx, HK_E_INVALID_ARG, "hk_terminal_greedy: NULL argument");
    if (n_valid == 0 || n_valid > lm_head->view.rows)
        return set_error(ctx, HK_E_GEOMETRY, "hk_terminal_greedy: need 0 < n_valid <= lm_head rows");
    if (!(eps >= 0.0f) || !std::isfinite(eps)) return set_error(ctx, HK_E_INVALID_ARG, "hk_terminal_greedy: bad eps");
    if (!aligned16(hidden)) return set_error(ctx, HK_E_INVALID_ARG, "hk_terminal_greedy: hidden must be 16-byte aligned");
    if (reinterpret_cast<uintptr_t>(pick) & 7u)
        return set_error(ctx, HK_E_INVALID_ARG, "hk_terminal_greedy: pick must be 8-byte aligned");
    return head_greedy(ctx, hidden, norm_w, eps, lm_head, n_valid, xn, logits, pick, token,
                       static_cast<hipStream_t>(stream));
}

extern "C" int hk_terminal_greedy_noalloc(hk_ctx* ctx, const float* hidden, const float* norm_w, float eps,
                                          const hk_organ* lm_head, uint32_t n_valid, int32_t* token,
                                          hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!lm_head || !hidden || !norm_w || !token)
        return set_error(ctx, HK_E_INVALID_ARG, "hk_terminal_greedy_noalloc: NULL argument");
    if (lm_head->view.rows > HK_NOALLOC_HEAD_MAX_ROWS || lm_head->view.cols > HK_NOALLOC_HEAD_MAX_COLS)
        return set_error(ctx, HK_E_UNSUPPORTED,
                         "hk_terminal_greedy_noalloc: lm_head above the workspace's " +
                             std::to_string(HK_NOALLOC_HEAD_MAX_ROWS) + " rows x " +
                             std::to_string(HK_NOALLOC_HEAD_MAX_COLS) + " cols");
    if (n_valid == 0 || n_valid > lm_head->view.rows)
        return set_error(ctx, HK_E_GEOMETRY, "hk_terminal_greedy_noalloc: need 0 < n_valid <= lm_head rows");
    if (!(eps >= 0.0f) || !std::isfinite(eps))
        return set_error(ctx, HK_E_INVALID_ARG, "hk_terminal_greedy_noalloc: bad eps");
    if (!aligned16(hidden))
        return set_error(ctx, HK_E_INVALID_ARG, "hk_terminal_greedy_noalloc: hidden must be 16-byte aligned");
    // [logits | xn | pick]: the pick slot is zero (static storage, and every
    // call leaves it zeroed)
    if (!ctx->noalloc) {
        const int st = noalloc_scratch(ctx, &ctx->noalloc);
        if (st != HK_OK) return st;
    }
    uint8_t* ws = ctx->noalloc;
    float* logits = reinterpret_cast<float*>(ws);
    float* xn = reinterpret_cast<float*>(ws + NOALLOC_LOGITS);
    uint64_t* pick = reinterpret_cast<uint64_t*>(ws + NOALLOC_LOGITS + NOALLOC_XN);
    return head_greedy(ctx, hidden, norm_w, eps, lm_head, n_valid, xn, logits, pick, token,
                       static_cast<hipStream_t>(stream));
}

// ====================================================================== routers

extern "C" int hk_router_softmax_topk(hk_ctx* ctx, const float* logits, uint32_t n_tokens, uint32_t n_experts,
                                      uint32_t top_k, float tie_eps, int renorm, int32_t* ids, float* weights,
                                      hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!logits || !ids || !weights) return set_error(ctx, HK_E_INVALID_ARG, "router: NULL pointer");
    if (n_tokens == 0 || n_experts == 0 || top_k == 0 || top_k > n_experts)
        return set_error(ctx, HK_E_INVALID_ARG, "router: need 0 < top_k <= n_experts and n_tokens > 0");
    if (n_experts > 8192 || top_k > 64) return set_error(ctx, HK_E_UNSUPPORTED, "router: n_experts above 8192 or top_k above 64");
    if (!(tie_eps >= 0.0f) || !std::isfinite(tie_eps)) return set_error(ctx, HK_E_INVALID_ARG, "router: tie_eps must be finite and >= 0");
    return check_hip(ctx,
                     launch_softmax_topk(logits, n_tokens, n_experts, top_k, tie_eps, renorm, ids, weights,
                                         ctx->dev_status, static_cast<hipStream_t>(stream)),
                     "router launch");
}

extern "C" int hk_router_noaux_tc(hk_ctx* ctx, const float* logits, const float* bias, uint32_t n_tokens,
                                  uint32_t n_experts, uint32_t n_group, uint32_t topk_group, uint32_t top_k,
                                  int norm_topk_prob, float routed_scaling_factor, int32_t* ids, float* weights,
                                  hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!logits || !bias || !ids || !weights) return set_error(ctx, HK_E_INVALID_ARG, "noaux_tc: NULL pointer");
    if (n_tokens == 0 || n_group == 0 || n_experts % n_group || topk_group == 0 || topk_group > n_group ||
        top_k == 0 || top_k > (n_experts / n_group) * topk_group)
        return set_error(ctx, HK_E_INVALID_ARG, "noaux_tc: inconsistent group / top-k geometry");
    if (n_experts > 8192 || top_k > 64) return set_error(ctx, HK_E_UNSUPPORTED, "noaux_tc: n_experts above 8192 or top_k above 64");
    return check_hip(ctx,
                     launch_noaux_tc(logits, bias, n_tokens, n_experts, n_group, topk_group, top_k, norm_topk_prob,
                                     routed_scaling_factor, ids, weights, static_cast<hipStream_t>(stream)),
                     "noaux_tc launch");
}

// ====================================================================== MoE model
// Expert organs are staged in the canonical layout (host upload or device
// generation) and repacked per layer into one slab of tiled organs; a device
// table of their views is indexed on the device by the route ids.

namespace {

constexpr uint32_t PROJ_NORM = 16, PROJ_ROUTER = 17, PROJ_SHARED_GATE = 18, PROJ_BIAS = 19, PROJ_COIN = 32;
constexpr float SIGMA_W = 0.02f, SIGMA_NORM = 0.02f, SIGMA_BIAS = 0.01f;
constexpr size_t MOE_LDS_LIMIT = 64 * 1024;
constexpr uint32_t MOE_MAX_SLOTS = 16;

struct MoeLayerHost {
    void* slab = nullptr;
    size_t slab_bytes = 0;
    size_t stride = 0;             // bytes between consecutive routed experts in the slab
    std::vector<OrganView> table;  // (E+1)*3
    std::vector<size_t> packed;    // per organ, algorithmic bytes
    OrganView* table_dev = nullptr;
    float* norm_w = nullptr;
    float* router_w = nullptr;
    float* gate_w = nullptr;
    float* bias = nullptr;
    bool ready = false;
};

}  // namespace

struct hk_moe_model {
    hk_moe_config cfg{};
    hk::MoeDims dims{};
    std::vector<MoeLayerHost> layers;
    void* dense = nullptr;   // norm/router/gate weights of all layers
    void* ws_mem = nullptr;
    void* tables = nullptr;  // device expert tables of all layers
    hk::MoeWs ws{};
    float* hbuf[2] = {nullptr, nullptr};
    // batched (noaux_tc) workspace for MOE_BATCH_MAX_TOKENS tokens (noaux_tc models)
    void* bws_mem = nullptr;
    uint32_t bws_tokens = 0;
    hk::MoeBatchWs bws{};
    // persistent decode (softmax models): per-layer descriptors on the device,
    // the flag-tagged hand-off words (every layer its own) and the next
    // launch's tag
    hk::MoeLayerDev* ldev = nullptr;
    void* stack_mem = nullptr;
    size_t stack_bytes = 0;
    hk::StackArgs st{};  // the buffer pointers and strides (per-call fields unset)
    uint32_t tag = 1;
    uint32_t stall_polls = HK_STALL_POLLS_DEFAULT;  // the persistent launch's bound on each wait
    int cu_count = 0;
};

// Per layer: norm weight [H], router [E x H], shared-expert gate [H], router bias [E].
static size_t dense_per_layer(const hk_moe_config& c) {
    return align256((size_t)c.hidden * 4) + align256((size_t)c.n_experts * c.hidden * 4) + align256((size_t)c.hidden * 4) +
           align256((size_t)c.n_experts * 4);
}

static void organ_shape(const hk_moe_config& c, uint32_t e, uint32_t p, uint32_t* rows, uint32_t* cols) {
    const uint32_t inter = e == c.n_experts ? c.shared_inter : c.inter;
    if (p < 2) {
        *rows = inter;
        *cols = c.hidden;
    } else {
        *rows = c.hidden;
        *cols = inter;
    }
}

extern "C" uint64_t hk_moe_stream_id(uint32_t layer, uint32_t expert, uint32_t proj) {
    return ((uint64_t)(layer + 1) << 40) | ((uint64_t)expert << 8) | (uint64_t)proj;
}

// The batched (noaux_tc) block's workspace for its largest batch
// (MOE_BATCH_MAX_TOKENS tokens), allocated with the model so that the
// compute call allocates nothing.
static int alloc_batch_ws(hk_ctx* ctx, hk_moe_model* m) {
    const hk_moe_config& c = m->cfg;
    const uint32_t T = hk::MOE_BATCH_MAX_TOKENS;
    const uint32_t imax = std::max(c.inter, c.shared_inter), K = c.top_k, E = c.n_experts;
    const uint32_t S = (c.hidden + hk::MOE_BATCH_ROUTER_COLS - 1) / hk::MOE_BATCH_ROUTER_COLS;
    const size_t pairs = (size_t)T * K + (c.shared_inter ? T : 0);
    const size_t xs = align256(moe_batch_img_bytes(c.hidden)), as = align256(moe_batch_img_bytes(imax));
    const size_t sz[] = {
        (size_t)T * xs,                    // ximg
        (size_t)T * 4,                     // ximg_e
        (size_t)S * T * E * 4,             // part
        (size_t)T * K * 4,                 // ids
        (size_t)T * K * 4,                 // w
        (size_t)T * K * 4,                 // rank
        ((size_t)E + 1) * 16,              // active
        4,                                 // n_active
        pairs * 4,                         // members
        pairs * imax * 4,                  // act
        pairs * as,                        // aimg
        pairs * 4,                         // aimg_e
        pairs * c.hidden * 4,              // ybuf
    };
    size_t total = 0;
    for (size_t b : sz) total += align256(b);
    if (hipMalloc(&m->bws_mem, total) != hipSuccess) return set_error(ctx, HK_E_NOMEM, "batched MoE workspace allocation failed");
    uint8_t* p = static_cast<uint8_t*>(m->bws_mem);
    void* ptr[sizeof(sz) / sizeof(sz[0])];
    for (size_t i = 0; i < sizeof(sz) / sizeof(sz[0]); ++i) {
        ptr[i] = p;
        p += align256(sz[i]);
    }
    hk::MoeBatchWs& w = m->bws;
    w.ximg = static_cast<uint8_t*>(ptr[0]);
    w.ximg_e = static_cast<int32_t*>(ptr[1]);
    w.part = static_cast<float*>(ptr[2]);
    w.ids = static_cast<int32_t*>(ptr[3]);
    w.w = static_cast<float*>(ptr[4]);
    w.rank = static_cast<int32_t*>(ptr[5]);
    w.active = static_cast<uint4*>(ptr[6]);
    w.n_active = static_cast<uint32_t*>(ptr[7]);
    w.members = static_cast<uint32_t*>(ptr[8]);
    w.act = static_cast<float*>(ptr[9]);
    w.aimg = static_cast<uint8_t*>(ptr[10]);
    w.aimg_e = static_cast<int32_t*>(ptr[11]);
    w.ybuf = static_cast<float*>(ptr[12]);
    w.ximg_stride = (uint32_t)xs;
    w.aimg_stride = (uint32_t)as;
    w.status = ctx->dev_status;
    m->bws_tokens = T;
    return HK_OK;
}

// Layer l's descriptor for the persistent decode (after the layer is set).
static int upload_ldev(hk_ctx* ctx, hk_moe_model* m, uint32_t l) {
    if (!m->ldev) return HK_OK;
    const MoeLayerHost& L = m->layers[l];
    const hk::MoeLayerDev d{L.norm_w, L.router_w, (m->cfg.shared_gate && m->cfg.shared_inter) ? L.gate_w : nullptr,
                            L.table_dev, L.stride};
    return check_hip(ctx, hipMemcpy(m->ldev + l, &d, sizeof d, hipMemcpyHostToDevice), "layer descriptor upload");
}

// The persistent decode's buffers (zeroed: tag 0 is never waited for).  The
// The persistent decode's hand-off words: per layer, h [H], the logits
// [E + 1] and the activations [slots x Imax], then RDY_REP replicas of each
// ready array (down tiles of H, route blocks, gate/up tiles x slots).  Every
// array starts on a 256-byte boundary; replicas are an odd number of
// 256-byte units apart so that they fall in different memory channels.
// About (8 (H + E + slots Imax) + 24 (tiles + blocks) RDY_REP) bytes a layer.
static int alloc_stack(hk_ctx* ctx, hk_moe_model* m) {
    const hk_moe_config& c = m->cfg;
    const uint32_t slots = c.top_k + (c.shared_inter ? 1u : 0u), imax = std::max(c.inter, c.shared_inter);
    const uint32_t gu_tiles = n_tiles_for(c.shared_inter ? imax : c.inter);
    auto words = [](size_t n) { return (uint32_t)((n + 31) / 32 * 32); };       // 256-byte units
    auto rstride = [&](size_t n) { return words(n) | 32u; };                   // odd number of units
    hk::StackArgs& a = m->st;
    a.hs = words(c.hidden);
    a.ls = words((size_t)c.n_experts + 1);
    a.as = words((size_t)slots * imax);
    a.hrs = rstride(n_tiles_for(c.hidden));
    a.lrs = rstride((size_t)c.n_experts / 4 + 2);
    a.ars = rstride((size_t)slots * gu_tiles);
    const size_t per_layer = (size_t)a.hs + a.ls + a.as + (size_t)hk::RDY_REP * (a.hrs + a.lrs + a.ars);
    m->stack_bytes = (per_layer * c.n_layers + 32) * 8;
    int cu = 0;
    if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, ctx->device) != hipSuccess)
        return set_error(ctx, HK_E_HIP, "hipDeviceGetAttribute (CU count)");
    m->cu_count = cu;
    if (hipMalloc(&m->ldev, (size_t)c.n_layers * sizeof(hk::MoeLayerDev)) != hipSuccess ||
        hipMalloc(&m->stack_mem, m->stack_bytes) != hipSuccess) {
        if (m->ldev) (void)hipFree(m->ldev);
        m->ldev = nullptr;
        m->stack_mem = nullptr;
        return set_error(ctx, HK_E_NOMEM, "persistent decode buffers: allocation failed");
    }
    if (hipMemset(m->stack_mem, 0, m->stack_bytes) != hipSuccess ||
        hipMemset(m->ldev, 0, (size_t)c.n_layers * sizeof(hk::MoeLayerDev)) != hipSuccess) {
        (void)hipFree(m->ldev);
        (void)hipFree(m->stack_mem);
        m->ldev = nullptr;
        m->stack_mem = nullptr;
        return set_error(ctx, HK_E_HIP, "persistent decode buffers: clear failed");
    }
    uint64_t* p = static_cast<uint64_t*>(m->stack_mem);
    const size_t L = c.n_layers;
    a.h = p;
    a.logits = a.h + L * a.hs;
    a.act = a.logits + L * a.ls;
    a.h_rdy = a.act + L * a.as;
    a.l_rdy = a.h_rdy + L * hk::RDY_REP * a.hrs;
    a.a_rdy = a.l_rdy + L * hk::RDY_REP * a.lrs;
    a.abort = reinterpret_cast<uint32_t*>(a.a_rdy + L * hk::RDY_REP * a.ars);
    return HK_OK;
}

extern "C" int hk_moe_model_create(hk_ctx* ctx, const hk_moe_config* cfg, hk_moe_model** out) {
    if (!ctx || !cfg || !out) return HK_E_INVALID_ARG;
    *out = nullptr;
    const hk_moe_config& c = *cfg;
    if (c.n_layers == 0 || c.hidden == 0 || c.inter == 0 || c.n_experts == 0 || c.top_k == 0 || c.top_k > c.n_experts)
        return set_error(ctx, HK_E_INVALID_ARG, "moe config: zero dimension or top_k > n_experts");
    if (c.expert_kind != HK_Q4 && c.expert_kind != HK_MIXED)
        return set_error(ctx, HK_E_UNSUPPORTED, "moe config: expert_kind must be HK_Q4 or HK_MIXED");
    const uint32_t slots = c.top_k + (c.shared_inter ? 1u : 0u);
    if (slots > MOE_MAX_SLOTS || c.n_experts > 4096 || c.hidden > 8192 || c.hidden % 128)
        return set_error(ctx, HK_E_UNSUPPORTED,
                         "moe config: need top_k (+1 shared) <= 16, n_experts <= 4096, hidden % 128 == 0, hidden <= 8192");
    if (c.router != HK_ROUTER_SOFTMAX && c.router != HK_ROUTER_NOAUX_TC)
        return set_error(ctx, HK_E_UNSUPPORTED, "moe config: router must be HK_ROUTER_SOFTMAX or HK_ROUTER_NOAUX_TC");
    if (c.router == HK_ROUTER_NOAUX_TC) {
        if (c.n_group == 0 || c.n_group > 64 || c.n_experts % c.n_group || c.topk_group == 0 || c.topk_group > c.n_group ||
            c.top_k > (c.n_experts / c.n_group) * c.topk_group)
            return set_error(ctx, HK_E_INVALID_ARG, "moe config: inconsistent noaux_tc group / top-k geometry");
        if (!std::isfinite(c.routed_scaling_factor))
            return set_error(ctx, HK_E_INVALID_ARG, "moe config: routed_scaling_factor must be finite");
        if (c.expert_kind != HK_Q4 || c.shared_gate || c.n_experts > hk::MOE_BATCH_MAX_EXPERTS)
            return set_error(ctx, HK_E_UNSUPPORTED,
                             "moe config: the noaux_tc block needs Q4 experts, no shared gate, n_experts <= 512");
    }
    const int grp = c.expert_kind == HK_MIXED ? 128 : c.expert_group;
    int rc = validate_shape(ctx, c.expert_kind, grp, c.inter, c.hidden);
    if (!rc) rc = validate_shape(ctx, c.expert_kind, grp, c.hidden, c.inter);
    if (!rc && c.shared_inter) rc = validate_shape(ctx, c.expert_kind, grp, c.hidden, c.shared_inter);
    if (rc) return rc;
    if (!(c.eps > 0.0f) || !std::isfinite(c.eps)) return set_error(ctx, HK_E_INVALID_ARG, "moe config: eps must be positive");
    if (!(c.route_tie_eps >= 0.0f) || !std::isfinite(c.route_tie_eps))
        return set_error(ctx, HK_E_INVALID_ARG, "moe config: route_tie_eps must be finite and >= 0");
    if (c.stack_launch != HK_STACK_PER_LAYER && c.stack_launch != HK_STACK_PERSISTENT)
        return set_error(ctx, HK_E_INVALID_ARG, "moe config: stack_launch must be HK_STACK_PER_LAYER or HK_STACK_PERSISTENT");
    const uint32_t imax = std::max(c.inter, c.shared_inter);
    if (c.router == HK_ROUTER_SOFTMAX && (moe_gate_up_lds_bytes(c.expert_kind, c.hidden) > MOE_LDS_LIMIT ||
                                          moe_route_lds_bytes(c.expert_kind, c.hidden) > MOE_LDS_LIMIT ||
                                          moe_down_lds_bytes(c.expert_kind, imax, slots) > MOE_LDS_LIMIT))
        return set_error(ctx, HK_E_UNSUPPORTED, "moe config: x images of hidden / intermediate exceed 64 KiB of LDS");
    hk_moe_model* m = new hk_moe_model();
    m->cfg = c;
    m->cfg.expert_group = grp;
    m->dims = hk::MoeDims{c.hidden,    c.inter, c.shared_inter, imax, c.n_experts, c.top_k, c.shared_inter ? 1 : 0,
                          c.eps,       c.route_tie_eps};
    m->layers.resize(c.n_layers);
    const size_t dpl = dense_per_layer(c);
    const size_t tab = align256((size_t)(c.n_experts + 1) * 3 * sizeof(OrganView));
    const size_t img = align256((size_t)c.hidden * 4);
    const size_t dnh = align256((size_t)slots * hk::moe_dn_hdr_stride(c.hidden, imax) * 16);
    const size_t ws = align256(((size_t)c.n_experts + 4) * 4) + 3 * 256 + align256((size_t)slots * imax * 4) + img + 256 +
                      2 * align256((size_t)c.hidden * 4) + dnh;
    if (hipMalloc(&m->dense, dpl * c.n_layers) != hipSuccess || hipMalloc(&m->tables, tab * c.n_layers) != hipSuccess ||
        hipMalloc(&m->ws_mem, ws) != hipSuccess) {
        if (m->dense) (void)hipFree(m->dense);
        if (m->tables) (void)hipFree(m->tables);
        if (m->ws_mem) (void)hipFree(m->ws_mem);
        delete m;
        return set_error(ctx, HK_E_NOMEM, "moe model allocation failed");
    }
    // zero tables (layers without weights select nothing) and the workspace
    if (hipMemset(m->tables, 0, tab * c.n_layers) != hipSuccess || hipMemset(m->ws_mem, 0, ws) != hipSuccess) {
        (void)hipFree(m->dense);
        (void)hipFree(m->tables);
        (void)hipFree(m->ws_mem);
        delete m;
        return set_error(ctx, HK_E_HIP, "moe model initialisation failed");
    }
    for (uint32_t l = 0; l < c.n_layers; ++l) {
        uint8_t* d = static_cast<uint8_t*>(m->dense) + l * dpl;
        MoeLayerHost& L = m->layers[l];
        L.norm_w = reinterpret_cast<float*>(d);
        L.router_w = reinterpret_cast<float*>(d + align256((size_t)c.hidden * 4));
        L.gate_w = reinterpret_cast<float*>(d + align256((size_t)c.hidden * 4) + align256((size_t)c.n_experts * c.hidden * 4));
        L.bias = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(L.gate_w) + align256((size_t)c.hidden * 4));
        L.table_dev = reinterpret_cast<OrganView*>(static_cast<uint8_t*>(m->tables) + l * tab);
        L.table.assign((size_t)(c.n_experts + 1) * 3, OrganView{});
        L.packed.assign((size_t)(c.n_experts + 1) * 3, 0);
    }
    uint8_t* w = static_cast<uint8_t*>(m->ws_mem);
    m->ws.logits = reinterpret_cast<float*>(w);
    w += align256(((size_t)c.n_experts + 4) * 4);
    m->ws.ids = reinterpret_cast<int32_t*>(w);
    w += 256;
    m->ws.weights = reinterpret_cast<float*>(w);
    w += 256;
    m->ws.gate = reinterpret_cast<float*>(w);
    w += 256;
    m->ws.act = reinterpret_cast<float*>(w);
    w += align256((size_t)slots * imax * 4);
    m->ws.xn = reinterpret_cast<float*>(w);
    w += img;
    w += 256;
    m->hbuf[0] = reinterpret_cast<float*>(w);
    w += align256((size_t)c.hidden * 4);
    m->hbuf[1] = reinterpret_cast<float*>(w);
    w += align256((size_t)c.hidden * 4);
    m->ws.dn_hdr = reinterpret_cast<uint4*>(w);
    m->ws.status = ctx->dev_status;
    if (c.router == HK_ROUTER_SOFTMAX && (rc = alloc_stack(ctx, m))) {
        (void)hipFree(m->dense);
        (void)hipFree(m->tables);
        (void)hipFree(m->ws_mem);
        delete m;
        return rc;
    }
    if (c.router == HK_ROUTER_NOAUX_TC && (rc = alloc_batch_ws(ctx, m))) {
        (void)hipFree(m->dense);
        (void)hipFree(m->tables);
        (void)hipFree(m->ws_mem);
        delete m;
        return rc;
    }
    *out = m;
    return HK_OK;
}

extern "C" int hk_moe_model_free(hk_ctx* ctx, hk_moe_model* m) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!m) return HK_OK;
    (void)hipDeviceSynchronize();
    for (auto& L : m->layers)
        if (L.slab) (void)hipFree(L.slab);
    (void)hipFree(m->dense);
    (void)hipFree(m->tables);
    (void)hipFree(m->ws_mem);
    if (m->bws_mem) (void)hipFree(m->bws_mem);
    if (m->ldev) (void)hipFree(m->ldev);
    if (m->stack_mem) (void)hipFree(m->stack_mem);
    delete m;
    return HK_OK;
}

// Repacks one layer's staged canonical organs (canon[i], mixed binary-group
// counts nbin[i]; organ i = expert i / 3, projection i % 3, expert
// n_experts = the shared one) into a fresh slab of tiled organs and uploads
// the layer's device table.  Routed experts sit at a uniform stride: each
// projection is placed with the layer's largest layout of it (mixed: the
// most Q2 groups), so routed expert e's views are expert 0's advanced by
// e * stride.  Synchronises `st`.
static int repack_layer(hk_ctx* ctx, MoeLayerHost& L, const std::vector<CanonView>& canon,
                        const std::vector<uint32_t>& nbin, uint32_t n_experts, hipStream_t st) {
    const size_t n_org = canon.size();
    const int kind = canon[0].kind;
    std::vector<uint32_t> nq2(n_org, 0);
    size_t words = 0, max_items = 0;
    uint32_t max_q2[3] = {0, 0, 0};
    for (size_t i = 0; i < n_org; ++i) {
        const CanonView& v = canon[i];
        const uint32_t nb = kind == HK_MIXED ? nbin[i] : 0;
        if (kind == HK_MIXED) nq2[i] = (uint32_t)((size_t)v.rows * v.cols / 128) - nb;
        (void)tiled_bytes(kind, v.group, v.rows, v.cols, nb, nq2[i], &L.packed[i]);
        if (i / 3 < n_experts) max_q2[i % 3] = std::max(max_q2[i % 3], nq2[i]);
        const size_t blocks = (size_t)n_tiles_for(v.rows) * n_steps_for(kind, v.cols);
        words += blocks;
        max_items = std::max(max_items, blocks * 64);
    }
    // the envelope layout of each routed projection, and the shared expert's own
    size_t off[3], stride = 0;
    uint32_t env_bin[3];
    for (int p = 0; p < 3; ++p) {
        const CanonView& v = canon[(size_t)p];
        const uint32_t groups = kind == HK_MIXED ? (uint32_t)((size_t)v.rows * v.cols / 128) : 0;
        env_bin[p] = groups - max_q2[p];
        off[p] = stride;
        stride += tiled_bytes(kind, v.group, v.rows, v.cols, env_bin[p], max_q2[p], nullptr);
    }
    size_t total = stride * n_experts;
    for (size_t i = (size_t)n_experts * 3; i < n_org; ++i)
        total += tiled_bytes(kind, canon[i].group, canon[i].rows, canon[i].cols, kind == HK_MIXED ? nbin[i] : 0, nq2[i],
                             nullptr);
    if (L.slab) {
        (void)hipStreamSynchronize(st);
        (void)hipFree(L.slab);
        L.slab = nullptr;
        L.slab_bytes = 0;
    }
    L.ready = false;
    if (hipMalloc(&L.slab, total) != hipSuccess) return set_error(ctx, HK_E_NOMEM, "expert slab allocation failed");
    L.slab_bytes = total;
    L.stride = stride;
    void* aux = nullptr;
    const size_t jobs_bytes = align256(n_org * sizeof(RepackJob));
    if (hipMalloc(&aux, jobs_bytes + words * 4 + 256) != hipSuccess) return set_error(ctx, HK_E_NOMEM, "repack job allocation failed");
    std::vector<RepackJob> jobs(n_org);
    uint8_t* slab = static_cast<uint8_t*>(L.slab);
    uint8_t* p_shared = slab + stride * n_experts;
    uint32_t* counts = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(aux) + jobs_bytes);
    for (size_t i = 0; i < n_org; ++i) {
        const CanonView& v = canon[i];
        const size_t e = i / 3, p = i % 3;
        if (e < n_experts) {
            L.table[i] = tiled_place(kind, v.group, v.rows, v.cols, kind == HK_MIXED ? env_bin[p] : 0,
                                     kind == HK_MIXED ? max_q2[p] : 0, slab + e * stride + off[p]);
        } else {
            L.table[i] = tiled_place(kind, v.group, v.rows, v.cols, kind == HK_MIXED ? nbin[i] : 0, nq2[i], p_shared);
            p_shared += tiled_bytes(kind, v.group, v.rows, v.cols, kind == HK_MIXED ? nbin[i] : 0, nq2[i], nullptr);
        }
        jobs[i] = RepackJob{v, L.table[i], counts};
        counts += (size_t)L.table[i].n_tiles * L.table[i].steps;
    }
    int rc = check_hip(ctx, hipMemcpyAsync(aux, jobs.data(), n_org * sizeof(RepackJob), hipMemcpyHostToDevice, st),
                       "repack job upload");
    if (!rc) rc = check_hip(ctx, launch_repack_batch(kind, static_cast<RepackJob*>(aux), (uint32_t)n_org, max_items, st),
                            "expert repack");
    if (!rc) rc = check_hip(ctx, hipMemcpyAsync(L.table_dev, L.table.data(), L.table.size() * sizeof(OrganView),
                                                hipMemcpyHostToDevice, st),
                            "expert table upload");
    if (!rc) rc = check_hip(ctx, hipStreamSynchronize(st), "hipStreamSynchronize (expert repack)");
    (void)hipFree(aux);
    return rc;
}

extern "C" int hk_moe_model_set_layer(hk_ctx* ctx, hk_moe_model* m, uint32_t layer, const hk_moe_layer_src* src,
                                      hk_stream stream) {
    if (!ctx || !m || !src) return HK_E_INVALID_ARG;
    const hk_moe_config& c = m->cfg;
    if (layer >= c.n_layers) return set_error(ctx, HK_E_INVALID_ARG, "layer index out of range");
    if (!src->norm_w || !src->router_w || !src->experts || (c.shared_inter && !src->shared) ||
        (c.shared_gate && c.shared_inter && !src->shared_gate_w) || (c.router == HK_ROUTER_NOAUX_TC && !src->router_bias))
        return set_error(ctx, HK_E_INVALID_ARG, "layer source: missing tensor (a missing tensor must raise, not zero-fill)");
    const uint32_t n_org = (c.n_experts + (c.shared_inter ? 1 : 0)) * 3;
    std::vector<Layout> lay(n_org);
    std::vector<const hk_organ_src*> srcs(n_org);
    size_t total = 0;
    for (uint32_t i = 0; i < n_org; ++i) {
        const uint32_t e = i / 3, p = i % 3;
        const hk_organ_src* s = e < c.n_experts ? &src->experts[i] : &src->shared[p];
        uint32_t rows, cols;
        organ_shape(c, e, p, &rows, &cols);
        if (s->kind != c.expert_kind || s->rows != rows || s->cols != cols ||
            (c.expert_kind == HK_Q4 && s->group != c.expert_group))
            return set_error(ctx, HK_E_GEOMETRY,
                             "expert " + std::to_string(e) + " proj " + std::to_string(p) + " disagrees with the model config");
        int rc = validate_src(ctx, s, &lay[i]);
        if (rc) return rc;
        srcs[i] = s;
        total += lay[i].total();
    }
    MoeLayerHost& L = m->layers[layer];
    hipStream_t st = static_cast<hipStream_t>(stream);
    void* stage = nullptr;
    if (hipMalloc(&stage, total) != hipSuccess) return set_error(ctx, HK_E_NOMEM, "expert staging allocation failed");
    std::vector<std::vector<uint32_t>> keep;
    std::vector<CanonView> canon(n_org);
    std::vector<uint32_t> nbin(n_org, 0);
    uint8_t* p = static_cast<uint8_t*>(stage);
    int rc = HK_OK;
    for (uint32_t i = 0; i < n_org && !rc; ++i) {
        rc = copy_src(ctx, srcs[i], lay[i], p, &canon[i], st, &keep);
        nbin[i] = srcs[i]->n_bin;
        p += lay[i].total();
    }
    if (!rc) rc = repack_layer(ctx, L, canon, nbin, c.n_experts, st);
    (void)hipStreamSynchronize(st);
    (void)hipFree(stage);
    if (rc) return rc;
    rc = check_hip(ctx, hipMemcpyAsync(L.norm_w, src->norm_w, (size_t)c.hidden * 4, hipMemcpyHostToDevice, st), "norm upload");
    if (!rc) rc = check_hip(ctx, hipMemcpyAsync(L.router_w, src->router_w, (size_t)c.n_experts * c.hidden * 4,
                                                hipMemcpyHostToDevice, st), "router upload");
    if (!rc && src->shared_gate_w)
        rc = check_hip(ctx, hipMemcpyAsync(L.gate_w, src->shared_gate_w, (size_t)c.hidden * 4, hipMemcpyHostToDevice, st),
                       "gate upload");
    if (!rc && src->router_bias)
        rc = check_hip(ctx, hipMemcpyAsync(L.bias, src->router_bias, (size_t)c.n_experts * 4, hipMemcpyHostToDevice, st),
                       "router bias upload");
    if (!rc) rc = check_hip(ctx, hipStreamSynchronize(st), "hipStreamSynchronize (layer upload)");
    if (rc) return rc;
    L.ready = true;
    rc = upload_ldev(ctx, m, layer);
    if (rc) return rc;
    return HK_OK;
}

extern "C" int hk_moe_model_fill_synthetic(hk_ctx* ctx, hk_moe_model* m, uint64_t seed, hk_stream stream) {
    if (!ctx || !m) return HK_E_INVALID_ARG;
    const hk_moe_config& c = m->cfg;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const uint32_t n_exp = c.n_experts + (c.shared_inter ? 1 : 0);
    const uint32_t n_org = n_exp * 3;
    void* jobs_dev = nullptr;
    void* aux = nullptr;
    if (hipMalloc(&jobs_dev, (size_t)std::max(n_org, 4u) * sizeof(SynthJob)) != hipSuccess ||
        hipMalloc(&aux, (size_t)n_org * 4 + 256) != hipSuccess) {
        if (jobs_dev) (void)hipFree(jobs_dev);
        return set_error(ctx, HK_E_NOMEM, "synthetic job table allocation failed");
    }
    uint32_t* counts = static_cast<uint32_t*>(aux);
    uint32_t* bad = counts + n_org;
    int rc = check_hip(ctx, hipMemsetAsync(bad, 0, 4, st), "memset");
    std::vector<SynthJob> jobs(n_org);
    std::vector<uint32_t> nbin(n_org, 0);
    std::vector<CanonView> canon(n_org);
    void* stage = nullptr;
    size_t stage_bytes = 0;
    for (uint32_t l = 0; l < c.n_layers && !rc; ++l) {
        MoeLayerHost& L = m->layers[l];
        // dense tensors
        SynthJob dj[4] = {};
        const uint32_t drows[4] = {1, c.n_experts, 1, 1};
        const uint32_t dcols[4] = {c.hidden, c.hidden, c.hidden, c.n_experts};
        const uint32_t dproj[4] = {PROJ_NORM, PROJ_ROUTER, PROJ_SHARED_GATE, PROJ_BIAS};
        float* dptr[4] = {L.norm_w, L.router_w, L.gate_w, L.bias};
        const float dsig[4] = {SIGMA_NORM, SIGMA_W, SIGMA_W, SIGMA_BIAS};
        for (int k = 0; k < 4; ++k) {
            dj[k].key = hk::stream_key(seed, hk_moe_stream_id(l, 0, dproj[k]));
            dj[k].sigma = dsig[k];
            dj[k].rows = drows[k];
            dj[k].cols = dcols[k];
            dj[k].dense = dptr[k];
        }
        rc = check_hip(ctx, hipMemcpyAsync(jobs_dev, dj, sizeof(dj), hipMemcpyHostToDevice, st), "job upload");
        if (!rc) rc = check_hip(ctx, launch_synth_jobs(HK_F32, static_cast<SynthJob*>(jobs_dev), 4,
                                                       (size_t)c.n_experts * c.hidden / 128 + 1, bad, st), "dense synth");
        if (!rc) rc = check_hip(ctx, hipStreamSynchronize(st), "sync");
        if (rc) break;
        // expert organs: keys and shapes
        size_t max_groups = 0;
        for (uint32_t i = 0; i < n_org; ++i) {
            const uint32_t e = i / 3, p = i % 3;
            uint32_t rows, cols;
            organ_shape(c, e, p, &rows, &cols);
            SynthJob& j = jobs[i];
            j = SynthJob{};
            j.key = hk::stream_key(seed, hk_moe_stream_id(l, e, p));
            j.coin_key = hk::stream_key(seed, hk_moe_stream_id(l, e, PROJ_COIN + p));
            j.sigma = SIGMA_W;
            j.group = c.expert_group;
            j.rows = rows;
            j.cols = cols;
            max_groups = std::max(max_groups, (size_t)rows * cols / (size_t)(c.expert_kind == HK_MIXED ? 128 : c.expert_group));
        }
        if (c.expert_kind == HK_MIXED) {
            rc = check_hip(ctx, hipMemcpyAsync(jobs_dev, jobs.data(), n_org * sizeof(SynthJob), hipMemcpyHostToDevice, st), "job upload");
            if (!rc) rc = check_hip(ctx, hipMemsetAsync(counts, 0, (size_t)n_org * 4, st), "memset");
            if (!rc) rc = check_hip(ctx, launch_synth_mixed_count(static_cast<SynthJob*>(jobs_dev), n_org, max_groups, counts, st),
                                    "mixed count");
            if (!rc) rc = check_hip(ctx, hipMemcpyAsync(nbin.data(), counts, (size_t)n_org * 4, hipMemcpyDeviceToHost, st), "count read");
            if (!rc) rc = check_hip(ctx, hipStreamSynchronize(st), "sync");
            if (rc) break;
        }
        // canonical staging for this layer
        std::vector<Layout> lay(n_org);
        size_t total = 0;
        for (uint32_t i = 0; i < n_org; ++i) {
            const SynthJob& j = jobs[i];
            const uint32_t groups = (uint32_t)((size_t)j.rows * j.cols / 128);
            lay[i] = layout_for(c.expert_kind, c.expert_group, j.rows, j.cols, nbin[i],
                                c.expert_kind == HK_MIXED ? groups - nbin[i] : 0);
            total += lay[i].total();
        }
        if (total > stage_bytes) {
            if (stage) (void)hipFree(stage);
            stage = nullptr;
            stage_bytes = 0;
            if (hipMalloc(&stage, total) != hipSuccess) {
                rc = set_error(ctx, HK_E_NOMEM, "expert staging allocation failed (layer " + std::to_string(l) + ")");
                break;
            }
            stage_bytes = total;
        }
        uint8_t* p = static_cast<uint8_t*>(stage);
        for (uint32_t i = 0; i < n_org; ++i) {
            SynthJob& j = jobs[i];
            CanonView v = place(c.expert_kind, c.expert_group, j.rows, j.cols, lay[i], p);
            j.scales = const_cast<uint16_t*>(v.scales);
            j.codes = const_cast<uint8_t*>(v.codes);
            j.tags = const_cast<uint8_t*>(v.tags);
            j.q2_scales = const_cast<uint16_t*>(v.q2_scales);
            j.q2_codes = const_cast<uint8_t*>(v.q2_codes);
            j.row_bin = const_cast<uint32_t*>(v.row_bin);
            j.row_q2 = const_cast<uint32_t*>(v.row_q2);
            canon[i] = v;
            p += lay[i].total();
        }
        rc = check_hip(ctx, hipMemcpyAsync(jobs_dev, jobs.data(), n_org * sizeof(SynthJob), hipMemcpyHostToDevice, st), "job upload");
        if (!rc) rc = check_hip(ctx, launch_synth_jobs(c.expert_kind, static_cast<SynthJob*>(jobs_dev), n_org, max_groups, bad, st),
                                "expert synth");
        if (!rc) rc = repack_layer(ctx, L, canon, nbin, c.n_experts, st);
        if (!rc) L.ready = true;
        if (!rc) rc = upload_ldev(ctx, m, l);
    }
    uint32_t badv = 0;
    if (!rc) rc = check_hip(ctx, hipMemcpyAsync(&badv, bad, 4, hipMemcpyDeviceToHost, st), "flag read");
    if (!rc) rc = check_hip(ctx, hipStreamSynchronize(st), "sync");
    (void)hipStreamSynchronize(st);
    if (stage) (void)hipFree(stage);
    (void)hipFree(jobs_dev);
    (void)hipFree(aux);
    if (!rc && badv) rc = set_error(ctx, HK_E_NONFINITE, "synthetic pack produced a non-finite scale");
    return rc;
}

extern "C" int hk_moe_model_bytes(const hk_moe_model* m, size_t* device_bytes, size_t* dense_bytes_per_layer) {
    if (!m) return HK_E_INVALID_ARG;
    size_t dev = 0;
    for (const auto& L : m->layers) dev += L.slab_bytes;
    dev += dense_per_layer(m->cfg) * m->cfg.n_layers;
    if (device_bytes) *device_bytes = dev;
    if (dense_bytes_per_layer)
        *dense_bytes_per_layer = (size_t)m->cfg.hidden * 4 * (1 + (m->cfg.shared_gate ? 1 : 0)) +
                                 (size_t)m->cfg.n_experts * m->cfg.hidden * 4;
    return HK_OK;
}

extern "C" int hk_moe_expert_bytes(const hk_moe_model* m, uint32_t layer, uint32_t expert, size_t* bytes) {
    if (!m || !bytes || layer >= m->cfg.n_layers || expert > m->cfg.n_experts) return HK_E_INVALID_ARG;
    const MoeLayerHost& L = m->layers[layer];
    if (expert == m->cfg.n_experts && !m->cfg.shared_inter) return HK_E_INVALID_ARG;
    *bytes = L.packed[expert * 3] + L.packed[expert * 3 + 1] + L.packed[expert * 3 + 2];
    return HK_OK;
}

static int moe_layer_dev(hk_ctx* ctx, hk_moe_model* m, uint32_t layer, MoeLayerDev* out) {
    if (layer >= m->cfg.n_layers) return set_error(ctx, HK_E_INVALID_ARG, "layer index out of range");
    MoeLayerHost& L = m->layers[layer];
    if (!L.ready) return set_error(ctx, HK_E_INVALID_ARG, "layer " + std::to_string(layer) + " has no weights");
    *out = MoeLayerDev{L.norm_w, L.router_w, (m->cfg.shared_gate && m->cfg.shared_inter) ? L.gate_w : nullptr,
                       L.table_dev, L.stride};
    return HK_OK;
}

extern "C" int hk_moe_decode_layer(hk_ctx* ctx, hk_moe_model* m, uint32_t layer, const float* h_in, float* h_out,
                                   int32_t* ids, float* weights, hk_stream stream) {
    if (!ctx || !m) return HK_E_INVALID_ARG;
    if (m->cfg.router != HK_ROUTER_SOFTMAX)
        return set_error(ctx, HK_E_UNSUPPORTED, "moe layer: the decode path routes with HK_ROUTER_SOFTMAX");
    if (!h_in || !h_out || h_in == h_out) return set_error(ctx, HK_E_INVALID_ARG, "moe layer: h_in/h_out NULL or aliased");
    if (!aligned16(h_in) || !aligned16(h_out)) return set_error(ctx, HK_E_INVALID_ARG, "moe layer: h_in/h_out must be 16-byte aligned");
    MoeLayerDev L;
    int rc = moe_layer_dev(ctx, m, layer, &L);
    if (rc) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    return check_hip(ctx, launch_moe_layer(m->cfg.expert_kind, m->dims, L, h_in, h_out, m->ws, ids, weights, st),
                     "moe layer launch");
}

// The persistent launch is selected per model (hk_moe_config.stack_launch);
// the default is the per-layer launches, which are faster at config-4 shapes.
static bool stack_enabled(const hk_moe_model* m) { return m->ldev && m->cfg.stack_launch == HK_STACK_PERSISTENT; }

extern "C" int hk_moe_model_set_stack_launch(hk_ctx* ctx, hk_moe_model* m, int32_t stack_launch) {
    if (!ctx || !m) return HK_E_INVALID_ARG;
    if (stack_launch != HK_STACK_PER_LAYER && stack_launch != HK_STACK_PERSISTENT)
        return set_error(ctx, HK_E_INVALID_ARG, "stack_launch must be HK_STACK_PER_LAYER or HK_STACK_PERSISTENT");
    m->cfg.stack_launch = stack_launch;
    return HK_OK;
}

static hk::StackArgs stack_args(hk_ctx* ctx, hk_moe_model* m, const float* h_in, float* h_out, int32_t* ids,
                                float* weights) {
    hk::StackArgs a = m->st;
    a.d = m->dims;
    a.layers = m->ldev;
    a.n_layers = m->cfg.n_layers;
    a.tag = m->tag;
    a.h_in = h_in;
    a.h_out = h_out;
    a.ids = ids;
    a.weights = weights;
    a.status = ctx->dev_status;
    a.gu_tiles = n_tiles_for(m->dims.has_shared ? std::max(m->dims.I, m->dims.SI) : m->dims.I);
    a.ng = a.gu_tiles * (m->dims.K + (m->dims.has_shared ? 1u : 0u));
    a.spin_limit = m->stall_polls;
    return a;
}

extern "C" int hk_moe_model_set_stall_polls(hk_ctx* ctx, hk_moe_model* m, uint32_t polls) {
    if (!ctx || !m) return HK_E_INVALID_ARG;
    m->stall_polls = polls;
    return HK_OK;
}

extern "C" int hk_moe_decode_stack_persistent(hk_ctx* ctx, hk_moe_model* m, int* persistent) {
    if (!ctx || !m || !persistent) return HK_E_INVALID_ARG;
    *persistent = 0;
    if (m->cfg.router != HK_ROUTER_SOFTMAX || !stack_enabled(m)) return HK_OK;
    bool fits = false;
    const hk::StackArgs a = stack_args(ctx, m, nullptr, nullptr, nullptr, nullptr);
    int rc = check_hip(ctx, launch_moe_stack(m->cfg.expert_kind, a, m->cu_count, nullptr, &fits, false),
                       "persistent decode check");
    if (rc) return rc;
    *persistent = fits ? 1 : 0;
    return HK_OK;
}

extern "C" int hk_moe_decode_stack(hk_ctx* ctx, hk_moe_model* m, const float* h_in, float* h_out, int32_t* ids,
                                   float* weights, hk_stream stream) {
    if (!ctx || !m) return HK_E_INVALID_ARG;
    if (m->cfg.router != HK_ROUTER_SOFTMAX)
        return set_error(ctx, HK_E_UNSUPPORTED, "moe stack: the decode path routes with HK_ROUTER_SOFTMAX");
    if (!h_in || !h_out) return set_error(ctx, HK_E_INVALID_ARG, "moe stack: NULL h_in/h_out");
    if (!aligned16(h_in) || !aligned16(h_out)) return set_error(ctx, HK_E_INVALID_ARG, "moe stack: h_in/h_out must be 16-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const uint32_t n = m->cfg.n_layers, K = m->cfg.top_k;
    for (uint32_t l = 0; l < n; ++l)
        if (!m->layers[l].ready) return set_error(ctx, HK_E_INVALID_ARG, "layer " + std::to_string(l) + " has no weights");
    // the whole token in one persistent launch when enabled and its grid can
    // be resident
    if (stack_enabled(m)) {
        if (m->tag > 0xF0000000u) {  // tags never wrap: clear the words and restart
            int rc = check_hip(ctx, launch_zero_words(static_cast<uint64_t*>(m->stack_mem), m->stack_bytes / 8, st),
                               "hand-off clear");
            if (rc) return rc;
            m->tag = 1;
        }
        hk::StackArgs a = stack_args(ctx, m, h_in, h_out, ids, weights);
        bool fits = false;
        int rc = check_hip(ctx, launch_moe_stack(m->cfg.expert_kind, a, m->cu_count, st, &fits), "persistent decode launch");
        if (rc) return rc;
        if (fits) {
            m->tag += 1;
            return HK_OK;
        }
    }
    const float* cur = h_in;
    for (uint32_t l = 0; l < n; ++l) {
        MoeLayerDev L;
        int rc = moe_layer_dev(ctx, m, l, &L);
        if (rc) return rc;
        float* dst = (l == n - 1) ? h_out : m->hbuf[l & 1];
        rc = check_hip(ctx,
                       launch_moe_layer(m->cfg.expert_kind, m->dims, L, cur, dst, m->ws, ids ? ids + (size_t)l * K : nullptr,
                                        weights ? weights + (size_t)l * K : nullptr, st),
                       "moe layer launch");
        if (rc) return rc;
        cur = dst;
    }
    return HK_OK;
}

extern "C" int hk_moe_block(hk_ctx* ctx, hk_moe_model* m, uint32_t layer, const int32_t* route_ids,
                            const float* route_weights, uint32_t n_routes, int include_shared, const float* x,
                            float* out, hk_stream stream) {
    if (!ctx || !m) return HK_E_INVALID_ARG;
    const hk_moe_config& c = m->cfg;
    if (!route_ids || !route_weights || !x || !out) return set_error(ctx, HK_E_INVALID_ARG, "moe block: NULL pointer");
    if (!aligned16(x) || !aligned16(out)) return set_error(ctx, HK_E_INVALID_ARG, "moe block: x/out must be 16-byte aligned");
    if (n_routes == 0 || n_routes > c.top_k)
        return set_error(ctx, HK_E_INVALID_ARG, "moe block: need 1 <= n_routes <= the model's top_k");
    MoeLayerDev L;
    int rc = moe_layer_dev(ctx, m, layer, &L);
    if (rc) return rc;
    const bool shared = include_shared && c.shared_inter;
    const uint32_t slots = n_routes + (shared ? 1u : 0u), imax = std::max(c.inter, c.shared_inter);
    if (moe_block_gate_up_lds_bytes(c.expert_kind, c.hidden) > MOE_LDS_LIMIT ||
        moe_down_lds_bytes(c.expert_kind, imax, slots) > MOE_LDS_LIMIT)
        return set_error(ctx, HK_E_UNSUPPORTED, "moe block: x images of hidden / intermediate exceed 64 KiB of LDS");
    hk::MoeDims d = m->dims;
    d.K = n_routes;
    d.has_shared = shared ? 1 : 0;
    return check_hip(ctx,
                     launch_moe_block(c.expert_kind, d, L, route_ids, route_weights, x, out, m->ws,
                                      static_cast<hipStream_t>(stream)),
                     "moe block launch");
}

extern "C" int hk_moe_forward_batch(hk_ctx* ctx, hk_moe_model* m, uint32_t layer, const uint16_t* x_bf16,
                                    uint32_t n_tokens, float* y, int32_t* ids, float* weights, hk_stream stream) {
    if (!ctx || !m) return HK_E_INVALID_ARG;
    const hk_moe_config& c = m->cfg;
    if (c.router != HK_ROUTER_NOAUX_TC)
        return set_error(ctx, HK_E_UNSUPPORTED, "moe batch: the batched block routes with HK_ROUTER_NOAUX_TC");
    if (n_tokens == 0 || n_tokens > hk::MOE_BATCH_MAX_TOKENS)
        return set_error(ctx, HK_E_INVALID_ARG, "moe batch: n_tokens must be in [1, 64]");
    if (!x_bf16 || !y || !aligned16(x_bf16) || !aligned16(y))
        return set_error(ctx, HK_E_INVALID_ARG, "moe batch: NULL x/y, or x/y not 16-byte aligned");
    MoeLayerDev L;
    int rc = moe_layer_dev(ctx, m, layer, &L);
    if (rc) return rc;
    hk::MoeBatchDims d{};
    d.T = n_tokens;
    d.H = c.hidden;
    d.I = c.inter;
    d.SI = c.shared_inter;
    d.Imax = std::max(c.inter, c.shared_inter);
    d.E = c.n_experts;
    d.K = c.top_k;
    d.n_group = c.n_group;
    d.topk_group = c.topk_group;
    d.norm_topk_prob = c.norm_topk_prob;
    d.scaling = c.routed_scaling_factor;
    d.S = (c.hidden + hk::MOE_BATCH_ROUTER_COLS - 1) / hk::MOE_BATCH_ROUTER_COLS;
    return check_hip(ctx,
                     launch_moe_batch(d, L, m->layers[layer].bias, x_bf16, y, m->bws, ids, weights,
                                      static_cast<hipStream_t>(stream)),
                     "moe batch launch");
}
