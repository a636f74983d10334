// api.hip — the extern "C" boundary of liblrs.so (declared in include/lrs.h).
#include "lrs_internal.h"

#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>

namespace lrs {

static thread_local std::string g_err;

void set_error(const std::string &msg) { g_err = msg; }

int fail(int code, const std::string &msg) {
    g_err = msg;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    g_err = std::string("HIP error: ") + hipGetErrorString(e) + " in " + what;
    return e == hipErrorOutOfMemory ? LRS_E_OOM : LRS_E_HIP;
}

// geometry check of gpu.rs:149-164: n_in multiple of the block, byte count
static int check_shape(uint32_t t, size_t len, uint32_t n_in, uint32_t n_out, bool need_len) {
    const int64_t be = block_elems(t), bb = block_bytes(t);
    if (be < 0) return fail(LRS_E_UNSUPPORTED, "unsupported ggml type " + std::to_string(t));
    if (n_in == 0 || n_out == 0) return fail(LRS_E_ARG, "empty tensor");
    if (n_in % (uint32_t)be != 0)
        return fail(LRS_E_ARG, "n_in=" + std::to_string(n_in) + " is not a multiple of the block size " +
                                   std::to_string(be));
    const size_t want = (size_t)(n_in / be) * (size_t)bb * n_out;
    if (need_len && len != want)
        return fail(LRS_E_ARG, "tensor has " + std::to_string(len) + " bytes, expected " +
                                   std::to_string(want) + " for " + std::to_string(n_out) + "x" +
                                   std::to_string(n_in));
    return LRS_OK;
}

static int alloc_weight(lrs_ctx *ctx, uint32_t t, uint32_t n_in, uint32_t n_out, lrs_weight **out) {
    lrs_weight *w = new lrs_weight();
    w->ctx = ctx;
    w->v.type = t;
    w->v.n_in = n_in;
    w->v.n_out = n_out;
    w->v.nb = n_in / (uint32_t)block_elems(t);
    w->q_alloc = weight_dev_bytes(t, n_in, n_out);
    hipError_t e = hipMalloc(&w->q, w->q_alloc);
    if (e != hipSuccess) {
        delete w;
        return hip_fail(e, "hipMalloc(weight)");
    }
    w->v.q = w->q;
    *out = w;
    return LRS_OK;
}

}  // namespace lrs

using namespace lrs;

// per-context device scratch of the entry points that need a staging buffer
// (input pack, host-buffer staging, GEMM operand planes).  Graphs captured on
// the context record its address, so while any of them is alive the buffer
// must not move: growth is refused instead (lrs_ctx::live_graphs).
struct lrs_ctx_scratch {
    void *p = nullptr;
    size_t n = 0;
};
static std::mutex g_scratch_mu;
static std::unordered_map<lrs_ctx *, lrs_ctx_scratch> g_scratch;

namespace lrs {
static int ctx_scratch(lrs_ctx *ctx, size_t bytes, void **p) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    lrs_ctx_scratch &s = g_scratch[ctx];
    if (s.n < bytes) {
        if (ctx->live_graphs > 0)
            return fail(LRS_E_ARG, "context scratch must grow to " + std::to_string(bytes) +
                                       " bytes but " + std::to_string(ctx->live_graphs) +
                                       " captured graph(s) still use it: destroy them first, or "
                                       "make the largest call before capturing");
        // growing frees the old buffer after a stream sync, which a stream
        // being captured into a graph cannot do
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(ctx->stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
            return hip_fail(hipErrorStreamCaptureUnsupported, "context scratch growth inside a capture");
        if (s.p) {
            hipError_t e = hipStreamSynchronize(ctx->stream);
            if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize(scratch)");
            (void)hipFree(s.p);
            s.p = nullptr;
            s.n = 0;
        }
        size_t n = bytes < (1u << 20) ? (1u << 20) : bytes;
        hipError_t e = hipMalloc(&s.p, n);
        if (e != hipSuccess) return hip_fail(e, "hipMalloc(scratch)");
        s.n = n;
    }
    *p = s.p;
    return LRS_OK;
}
}  // namespace lrs

// ---- input pack of lrs_matvec_dev_noalloc ---------------------------------
// A static device array instead of the context scratch: the pack of one
// column of an input of up to LRS_NOALLOC_MAX_N_IN elements (3.5 bytes per
// element, fully rewritten by every call, so nothing has to start at zero).
// Each GPU holds its own copy until the process ends.  In host code `scratch`
// only names the symbol: the device address of each GPU's copy comes from
// hipGetSymbolAddress, resolved once per device by the first
// lrs_matvec_dev_noalloc call there (so no other entry point depends on it).
static constexpr size_t NOALLOC_PACK_BYTES = 160 * 1024;
static __device__ __align__(256) uint8_t scratch[NOALLOC_PACK_BYTES];
static constexpr int NOALLOC_MAX_DEVICES = 64;
static std::mutex g_noalloc_mu;
static void *g_noalloc_ptr[NOALLOC_MAX_DEVICES];

namespace lrs {
// with `device` current: the device address of this GPU's `scratch`
static int noalloc_init(int device) {
    if (device < 0 || device >= NOALLOC_MAX_DEVICES)
        return fail(LRS_E_UNSUPPORTED, "the no-allocation matvec serves device indices 0.." +
                                           std::to_string(NOALLOC_MAX_DEVICES - 1));
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (g_noalloc_ptr[device]) return LRS_OK;
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(LRS_E_HIP, "hipGetSymbolAddress(scratch) returned a null address");
    g_noalloc_ptr[device] = p;
    return LRS_OK;
}
// with `device` current: the resolved address, resolving it on first use
static int noalloc_ptr(int device, void **p) {
    if (int rc = noalloc_init(device)) return rc;
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    *p = g_noalloc_ptr[device];
    return LRS_OK;
}
}  // namespace lrs

#define SETDEV(ctx) LRS_HIP(hipSetDevice((ctx)->device))

extern "C" {

const char *lrs_last_error(void) { return g_err.c_str(); }

const char *lrs_version(void) { return "lrs 0.1 gfx950"; }

int lrs_ctx_create(int device, lrs_ctx **out) {
    if (!out) return fail(LRS_E_ARG, "null out");
    int n = 0;
    LRS_HIP(hipGetDeviceCount(&n));
    if (n == 0) return fail(LRS_E_HIP, "no HIP device");
    if (device < 0) {
        size_t best = 0;
        device = 0;
        for (int i = 0; i < n; i++) {
            size_t fr = 0, tot = 0;
            if (hipSetDevice(i) == hipSuccess && hipMemGetInfo(&fr, &tot) == hipSuccess && fr > best) {
                best = fr;
                device = i;
            }
        }
    }
    if (device >= n) return fail(LRS_E_ARG, "device " + std::to_string(device) + " out of range");
    LRS_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    LRS_HIP(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(LRS_E_UNSUPPORTED, std::string("liblrs is built for gfx950, device is ") +
                                           prop.gcnArchName);
    lrs_ctx *c = new lrs_ctx();
    c->device = device;
    hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreate(&c->ev0);
    if (e == hipSuccess) e = hipEventCreate(&c->ev1);
    if (e != hipSuccess) {
        delete c;
        return hip_fail(e, "stream/event create");
    }
    *out = c;
    return LRS_OK;
}

void lrs_ctx_destroy(lrs_ctx *ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        auto it = g_scratch.find(ctx);
        if (it != g_scratch.end()) {
            if (it->second.p) (void)hipFree(it->second.p);
            g_scratch.erase(it);
        }
    }
    (void)hipEventDestroy(ctx->ev0);
    (void)hipEventDestroy(ctx->ev1);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

int lrs_ctx_sync(lrs_ctx *ctx) {
    if (!ctx) return fail(LRS_E_ARG, "null ctx");
    SETDEV(ctx);
    LRS_HIP(hipStreamSynchronize(ctx->stream));
    return LRS_OK;
}

int lrs_ctx_mem_info(lrs_ctx *ctx, size_t *free_bytes, size_t *total_bytes) {
    if (!ctx) return fail(LRS_E_ARG, "null ctx");
    SETDEV(ctx);
    size_t f = 0, t = 0;
    LRS_HIP(hipMemGetInfo(&f, &t));
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
    return LRS_OK;
}

int lrs_weight_upload(lrs_ctx *ctx, uint32_t t, const void *bytes, size_t len, uint32_t n_in,
                      uint32_t n_out, lrs_weight **out) {
    if (!ctx || !bytes || !out) return fail(LRS_E_ARG, "null argument");
    int rc = check_shape(t, len, n_in, n_out, true);
    if (rc) return rc;
    SETDEV(ctx);
    lrs_weight *w = nullptr;
    rc = alloc_weight(ctx, t, n_in, n_out, &w);
    if (rc) return rc;
    hipError_t e;
    if (!is_tiled(t)) {
        e = hipMemcpyAsync(w->q, bytes, len, hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    } else {
        // GGUF bytes to a staging buffer, then repacked into the tiled layout
        uint8_t *tmp = nullptr;
        e = hipMalloc(&tmp, len);
        if (e == hipSuccess) e = hipMemcpyAsync(tmp, bytes, len, hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess) e = launch_repack_from_gguf(tmp, w->v, w->q, ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (tmp) (void)hipFree(tmp);
    }
    if (e != hipSuccess) {
        lrs_weight_free(w);
        return hip_fail(e, "weight upload");
    }
    *out = w;
    return LRS_OK;
}

int lrs_weight_generate(lrs_ctx *ctx, uint32_t t, uint64_t seed, int mode, float d_lo, float d_hi,
                        uint32_t n_in, uint32_t n_out, lrs_weight **out) {
    if (!ctx || !out) return fail(LRS_E_ARG, "null argument");
    if (t != T_Q8_0 && t != T_Q4_K && t != T_Q5_K && t != T_Q6_K)
        return fail(LRS_E_UNSUPPORTED, "synthetic blocks exist for Q8_0/Q4_K/Q5_K/Q6_K only");
    int rc = check_shape(t, 0, n_in, n_out, false);
    if (rc) return rc;
    SETDEV(ctx);
    lrs_weight *w = nullptr;
    rc = alloc_weight(ctx, t, n_in, n_out, &w);
    if (rc) return rc;
    hipError_t e = launch_generate(w->v, w->q, seed, mode, d_lo, d_hi, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        lrs_weight_free(w);
        return hip_fail(e, "weight generate");
    }
    *out = w;
    return LRS_OK;
}

size_t lrs_weight_gguf_bytes(const lrs_weight *w) {
    if (!w) return 0;
    return (size_t)w->v.nb * w->v.n_out * (size_t)block_bytes(w->v.type);
}

int lrs_weight_download(lrs_ctx *ctx, const lrs_weight *w, void *dst, size_t len) {
    if (!ctx || !w || !dst) return fail(LRS_E_ARG, "null argument");
    if (len != lrs_weight_gguf_bytes(w)) return fail(LRS_E_ARG, "download size mismatch");
    SETDEV(ctx);
    if (!is_tiled(w->v.type)) {
        LRS_HIP(hipMemcpyAsync(dst, w->q, len, hipMemcpyDeviceToHost, ctx->stream));
        LRS_HIP(hipStreamSynchronize(ctx->stream));
        return LRS_OK;
    }
    uint8_t *tmp = nullptr;
    LRS_HIP(hipMalloc(&tmp, len));
    hipError_t e = launch_repack_to_gguf(w->v, tmp, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(dst, tmp, len, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    (void)hipFree(tmp);
    if (e != hipSuccess) return hip_fail(e, "weight download");
    return LRS_OK;
}

void lrs_weight_free(lrs_weight *w) {
    if (!w) return;
    (void)hipSetDevice(w->ctx->device);
    (void)hipStreamSynchronize(w->ctx->stream);
    if (w->q) (void)hipFree(w->q);
    delete w;
}

int lrs_dequant_f32(lrs_ctx *ctx, uint32_t t, const void *bytes, size_t len, float *out) {
    if (!ctx || !bytes || !out) return fail(LRS_E_ARG, "null argument");
    const int64_t be = block_elems(t), bb = block_bytes(t);
    if (be < 0) return fail(LRS_E_UNSUPPORTED, "unsupported ggml type " + std::to_string(t));
    if (len == 0 || len % (size_t)bb != 0)
        return fail(LRS_E_ARG, "byte count " + std::to_string(len) + " is not a multiple of the block size " +
                                   std::to_string(bb));
    const size_t nblk = len / (size_t)bb;
    if (nblk * (size_t)be > 0xFFFFFFFFull) return fail(LRS_E_ARG, "tensor too large for one call");
    lrs_weight *w = nullptr;
    int rc = lrs_weight_upload(ctx, t, bytes, len, (uint32_t)(nblk * be), 1, &w);
    if (rc) return rc;
    float *dev = nullptr;
    hipError_t e = hipMalloc(&dev, nblk * be * sizeof(float));
    if (e == hipSuccess) e = launch_dequant(w->v, dev, ctx->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(out, dev, nblk * be * sizeof(float), hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (dev) (void)hipFree(dev);
    lrs_weight_free(w);
    if (e != hipSuccess) return hip_fail(e, "dequant");
    return LRS_OK;
}

int lrs_weight_dequant_dev(lrs_ctx *ctx, const lrs_weight *w, float *out_dev) {
    if (!ctx || !w || !out_dev) return fail(LRS_E_ARG, "null argument");
    SETDEV(ctx);
    LRS_HIP(launch_dequant(w->v, out_dev, ctx->stream));
    return LRS_OK;
}

static int matvec_check(const lrs_weight *w, uint32_t cols) {
    if (cols == 0) return fail(LRS_E_ARG, "cols must be >= 1");
    const uint32_t t = w->v.type;
    if (t != T_Q8_0 && t != T_Q4_K && t != T_Q5_K && t != T_Q6_K)
        return fail(LRS_E_UNSUPPORTED, "matvec supports Q8_0/Q4_K/Q5_K/Q6_K weights");
    return LRS_OK;
}

int lrs_matvec_dev(lrs_ctx *ctx, const lrs_weight *w, const float *x_dev, float *y_dev,
                   uint32_t cols) {
    if (!ctx || !w || !x_dev || !y_dev) return fail(LRS_E_ARG, "null argument");
    int rc = matvec_check(w, cols);
    if (rc) return rc;
    SETDEV(ctx);
    void *pack = nullptr;  // only the staged form needs one
    if (!matvec_packs_in_kernel(w->v, cols))
        if (int rc_ = ctx_scratch(ctx, xpack_bytes(pack_blocks(w->v.type, w->v.n_in)), &pack))
            return rc_;
    LRS_HIP(launch_matvec(w->v, x_dev, y_dev, cols, pack, ctx->stream));
    return LRS_OK;
}

int lrs_matvec_dev_noalloc(lrs_ctx *ctx, const lrs_weight *w, const float *x_dev, float *y_dev,
                           uint32_t cols) {
    if (!ctx || !w || !x_dev || !y_dev) return fail(LRS_E_ARG, "null argument");
    int rc = matvec_check(w, cols);
    if (rc) return rc;
    const size_t need = xpack_bytes(pack_blocks(w->v.type, w->v.n_in));
    if (w->v.n_in > LRS_NOALLOC_MAX_N_IN || need > NOALLOC_PACK_BYTES)
        return fail(LRS_E_ARG, "n_in=" + std::to_string(w->v.n_in) +
                                   " is above the no-allocation matvec's maximum of " +
                                   std::to_string(LRS_NOALLOC_MAX_N_IN));
    SETDEV(ctx);
    void *pack = nullptr;
    if (int rc_ = noalloc_ptr(ctx->device, &pack)) return rc_;
    LRS_HIP(launch_matvec_staged(w->v, x_dev, y_dev, cols, pack, ctx->stream));
    return LRS_OK;
}

int lrs_quantize_q8_0_dev(lrs_ctx *ctx, const float *x_dev, uint32_t n, int half_even,
                          uint8_t *q8_dev) {
    if (!ctx || !x_dev || !q8_dev) return fail(LRS_E_ARG, "null argument");
    if (n == 0 || n % 32) return fail(LRS_E_ARG, "n must be a positive multiple of 32");
    SETDEV(ctx);
    LRS_HIP(launch_q8act(x_dev, n, n / 32, half_even ? 1 : 0, q8_dev, XPack{nullptr, nullptr},
                         ctx->stream));
    return LRS_OK;
}

int lrs_matvec_q8_0_actq_dev(lrs_ctx *ctx, const lrs_weight *w, const float *x_dev,
                             float *y_dev, uint32_t cols, int half_even) {
    if (!ctx || !w || !x_dev || !y_dev) return fail(LRS_E_ARG, "null argument");
    if (cols == 0) return fail(LRS_E_ARG, "cols must be >= 1");
    if (w->v.type != T_Q8_0)
        return fail(LRS_E_UNSUPPORTED, "the int8-activation matvec takes Q8_0 weights");
    SETDEV(ctx);
    void *pack = nullptr;
    if (int rc_ = ctx_scratch(ctx, xpack_bytes(pack_blocks(w->v.type, w->v.n_in)), &pack)) return rc_;
    LRS_HIP(launch_matvec_actq(w->v, x_dev, y_dev, cols, pack, half_even ? 1 : 0, ctx->stream));
    return LRS_OK;
}

int lrs_matvec_f32(lrs_ctx *ctx, const lrs_weight *w, const float *x, float *y, uint32_t cols) {
    if (!ctx || !w || !x || !y) return fail(LRS_E_ARG, "null argument");
    int rc = matvec_check(w, cols);
    if (rc) return rc;
    SETDEV(ctx);
    const size_t xb = (size_t)cols * w->v.n_in * sizeof(float);
    const size_t yb = (size_t)cols * w->v.n_out * sizeof(float);
    const size_t pb =
        matvec_packs_in_kernel(w->v, cols) ? 0 : xpack_bytes(pack_blocks(w->v.type, w->v.n_in));
    auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
    void *buf = nullptr;
    if (int rc_ = ctx_scratch(ctx, up(xb) + up(yb) + pb, &buf)) return rc_;
    float *xd = (float *)buf;
    float *yd = (float *)((char *)buf + up(xb));
    void *pack = pb ? (char *)buf + up(xb) + up(yb) : nullptr;
    LRS_HIP(hipMemcpyAsync(xd, x, xb, hipMemcpyHostToDevice, ctx->stream));
    LRS_HIP(launch_matvec(w->v, xd, yd, cols, pack, ctx->stream));
    LRS_HIP(hipMemcpyAsync(y, yd, yb, hipMemcpyDeviceToHost, ctx->stream));
    LRS_HIP(hipStreamSynchronize(ctx->stream));
    return LRS_OK;
}

int lrs_gemm_dev(lrs_ctx *ctx, const lrs_weight *w, const float *a_dev, float *y_dev, uint32_t m,
                 int precision) {
    if (!ctx || !w || !a_dev || !y_dev) return fail(LRS_E_ARG, "null argument");
    if (m == 0) return fail(LRS_E_ARG, "m must be >= 1");
    if (precision != 1 && precision != 3) return fail(LRS_E_ARG, "precision must be 1 or 3");
    if (w->v.type != T_Q4_K && w->v.type != T_Q5_K && w->v.type != T_Q6_K && w->v.type != T_Q8_0)
        return fail(LRS_E_UNSUPPORTED, "the GEMM supports Q4_K, Q5_K, Q6_K and Q8_0 weights");
    if (w->v.n_in % 256)
        return fail(LRS_E_ARG, "the GEMM needs n_in to be a multiple of 256");
    SETDEV(ctx);
    // the activation as bf16 planes (hi, and lo for precision 3) in context scratch
    // (and the K-slice partials when the GEMM is split over K)
    const size_t n = (size_t)m * w->v.n_in, ab = (n * 2 * (precision == 3 ? 2 : 1) + 255) & ~(size_t)255;
    const size_t wb = gemm_work_bytes(m, w->v.n_out, w->v.n_in, precision);
    void *buf = nullptr;
    if (int rc_ = ctx_scratch(ctx, ab + wb, &buf)) return rc_;
    __bf16 *hi = (__bf16 *)buf, *lo = precision == 3 ? hi + n : nullptr;
    LRS_HIP(launch_split_bf16(a_dev, n, hi, lo, ctx->stream));
    LRS_HIP(launch_gemm(w->v, hi, lo, y_dev, m, w->v.n_out, precision, ctx->stream, false,
                        wb ? (float *)((char *)buf + ab) : nullptr));
    return LRS_OK;
}

int lrs_gemm_group_dev(lrs_ctx *ctx, const lrs_weight *const *w, uint32_t n_w, const float *a_dev,
                       float *const *y_dev, uint32_t m, int precision) {
    if (!ctx || !w || !a_dev || !y_dev) return fail(LRS_E_ARG, "null argument");
    if (n_w == 0 || n_w > 3) return fail(LRS_E_ARG, "1 to 3 weights per group");
    if (m == 0) return fail(LRS_E_ARG, "m must be >= 1");
    if (precision != 1 && precision != 3) return fail(LRS_E_ARG, "precision must be 1 or 3");
    WeightView wv[3];
    uint32_t ldy[3];
    for (uint32_t i = 0; i < n_w; i++) {
        if (!w[i] || !y_dev[i]) return fail(LRS_E_ARG, "null weight or output");
        wv[i] = w[i]->v;
        ldy[i] = w[i]->v.n_out;
        if (wv[i].n_in != wv[0].n_in) return fail(LRS_E_ARG, "the weights of a group share n_in");
    }
    if (wv[0].n_in % 256) return fail(LRS_E_ARG, "the GEMM needs n_in to be a multiple of 256");
    if (!gemm_segs_supported(wv, n_w))
        return fail(LRS_E_UNSUPPORTED, "group types: one type, or Q4_K / Q5_K weights then Q6_K");
    SETDEV(ctx);
    const size_t n = (size_t)m * wv[0].n_in, ab = n * 2 * (precision == 3 ? 2 : 1);
    void *buf = nullptr;
    if (int rc_ = ctx_scratch(ctx, ab, &buf)) return rc_;
    __bf16 *hi = (__bf16 *)buf, *lo = precision == 3 ? hi + n : nullptr;
    LRS_HIP(launch_split_bf16(a_dev, n, hi, lo, ctx->stream));
    LRS_HIP(launch_gemm_segs(wv, y_dev, ldy, n_w, hi, lo, m, precision, ctx->stream));
    return LRS_OK;
}

int lrs_matvec_set_geom(int tiles_per_wave, int tile_groups, int k_slices) {
    if (set_matvec_geom(tiles_per_wave, tile_groups, k_slices) != 0)
        return fail(LRS_E_ARG, "unsupported matvec launch shape (tiles_per_wave, tile_groups, "
                               "k_slices); all 0 restores the automatic choice");
    return LRS_OK;
}

int lrs_dev_alloc(lrs_ctx *ctx, size_t bytes, void **dptr) {
    if (!ctx || !dptr) return fail(LRS_E_ARG, "null argument");
    SETDEV(ctx);
    LRS_HIP(hipMalloc(dptr, bytes ? bytes : 1));
    return LRS_OK;
}

int lrs_dev_free(lrs_ctx *ctx, void *dptr) {
    if (!ctx) return fail(LRS_E_ARG, "null ctx");
    SETDEV(ctx);
    LRS_HIP(hipStreamSynchronize(ctx->stream));
    if (dptr) LRS_HIP(hipFree(dptr));
    return LRS_OK;
}

int lrs_copy_h2d(lrs_ctx *ctx, void *dst_dev, const void *src, size_t bytes) {
    if (!ctx || (bytes && (!dst_dev || !src))) return fail(LRS_E_ARG, "null argument");
    SETDEV(ctx);
    LRS_HIP(hipMemcpyAsync(dst_dev, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    LRS_HIP(hipStreamSynchronize(ctx->stream));
    return LRS_OK;
}

int lrs_copy_d2h(lrs_ctx *ctx, void *dst, const void *src_dev, size_t bytes) {
    if (!ctx || (bytes && (!dst || !src_dev))) return fail(LRS_E_ARG, "null argument");
    SETDEV(ctx);
    LRS_HIP(hipMemcpyAsync(dst, src_dev, bytes, hipMemcpyDeviceToHost, ctx->stream));
    LRS_HIP(hipStreamSynchronize(ctx->stream));
    return LRS_OK;
}

// ---- graph capture of the asynchronous (*_dev) entry points ----
struct lrs_graph {
    lrs_ctx *ctx;
    hipGraphExec_t exec;
};

int lrs_capture_begin(lrs_ctx *ctx) {
    if (!ctx) return fail(LRS_E_ARG, "null ctx");
    SETDEV(ctx);
    LRS_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    return LRS_OK;
}

int lrs_capture_end(lrs_ctx *ctx, lrs_graph **out) {
    if (!ctx || !out) return fail(LRS_E_ARG, "null argument");
    SETDEV(ctx);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &g);
    if (e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return hip_fail(e, "hipStreamEndCapture (a call inside the capture failed or synchronised?)");
    }
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        ctx->live_graphs++;
    }
    *out = new lrs_graph{ctx, x};
    return LRS_OK;
}

int lrs_graph_launch(lrs_graph *g) {
    if (!g) return fail(LRS_E_ARG, "null graph");
    SETDEV(g->ctx);
    LRS_HIP(hipGraphLaunch(g->exec, g->ctx->stream));
    return LRS_OK;
}

void lrs_graph_destroy(lrs_graph *g) {
    if (!g) return;
    (void)hipSetDevice(g->ctx->device);
    (void)hipStreamSynchronize(g->ctx->stream);
    (void)hipGraphExecDestroy(g->exec);
    {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        g->ctx->live_graphs--;
    }
    delete g;
}

int lrs_timer_start(lrs_ctx *ctx) {
    if (!ctx) return fail(LRS_E_ARG, "null ctx");
    SETDEV(ctx);
    LRS_HIP(hipEventRecord(ctx->ev0, ctx->stream));
    return LRS_OK;
}

int lrs_timer_stop(lrs_ctx *ctx, float *ms) {
    if (!ctx || !ms) return fail(LRS_E_ARG, "null argument");
    SETDEV(ctx);
    LRS_HIP(hipEventRecord(ctx->ev1, ctx->stream));
    LRS_HIP(hipEventSynchronize(ctx->ev1));
    LRS_HIP(hipEventElapsedTime(ms, ctx->ev0, ctx->ev1));
    return LRS_OK;
}

}  // extern "C"
