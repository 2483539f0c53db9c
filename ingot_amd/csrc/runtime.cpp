// Host runtime of libingot_rocm: sessions, device pool, constant-weight packs
// and the kernel-layer entry points of include/ingot_rocm.h.
//
// A session is the ROCm counterpart of the Metal GPUSession's device state
// (graph/gpu_darwin_arm64.go:96-148): one HIP stream, a size-classed device
// pool for op outputs (tensor.Pool, tensor/pool.go:10-60), a growable
// workspace for packed activations, and the table of
// packed constant weights (bCache / bf16Packs / bWeights:
// ops/matmul.go:200-280, ops/quant.go:803-829).

#include "runtime.hpp"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>

using namespace ingot;

// Fixed device scratch of ingot_rocm_gemm_noalloc: the packed activations
// (bf16 / hi-lo planes, the decode GEMV's x planes, the int8 GEMV's
// quantised x) that ingot_rocm_gemm keeps in the session's growable
// workspace. Each device holds its own copy for the life of the process. In
// host code `scratch` only names the symbol: its device address comes from
// hipGetSymbolAddress, once per device (NoAllocDevice::addr), and only that
// address is handed to kernels.
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;

// Per device: the scratch array's address, and the ordering of the no-alloc
// calls that share it. Sessions run on their own streams and calls return
// before their kernels finish, so each call records `done` on its stream and
// a call from another session first makes its stream wait for it: the
// device's no-alloc calls run one after another in the order the host made
// them, whichever sessions they come from. Set up when a session first opens
// on the device (nothing is created in the call itself).
struct NoAllocDevice {
    void* addr = nullptr;
    hipEvent_t done = nullptr;
    const ingot_rocm_session* last = nullptr;  // session of the last recorded call
    std::mutex mu;                             // orders the calls on the host
};
static std::mutex g_scratch_mu;
static NoAllocDevice g_noalloc[kMaxDevices];

namespace {

thread_local std::string g_err;

inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

int elem_size(int dt) {
    switch (dt) {
        case INGOT_DT_F32:
        case INGOT_DT_I32: return 4;
        case INGOT_DT_F16:
        case INGOT_DT_BF16:
        case INGOT_DT_I16: return 2;
        case INGOT_DT_I8:
        case INGOT_DT_U8:
        case INGOT_DT_BOOL: return 1;
        case INGOT_DT_I64: return 8;
    }
    return 0;
}

// Operand bytes above which a GEMM's operands are taken not to stay in the
// Infinity Cache between uses: half of its 256 MB on MI355X.
constexpr int64_t kCacheResidentBytes = (int64_t)128 << 20;

// elements of a kind per 128-byte k-tile
int ktile_elems(GemmKind k) { return k == KIND_F32 ? 32 : (k == KIND_I8 ? 128 : 64); }
int kind_size(GemmKind k) { return k == KIND_F32 ? 4 : (k == KIND_I8 || k == KIND_I8G ? 1 : 2); }

// Picks the tile configuration with the least estimated time: full rounds of
// num_cus·occupancy workgroups, each round as long as the most loaded CU.
// Deep-ring entries marked one_round apply only when a single round holds
// every tile. force >= 0 (INGOT_GEMM_CFG) picks that entry when it exists.
int pick_config(GemmKind kind, int64_t M, int64_t N, int64_t batch, int num_cus, int force) {
    const GemmConfig* c;
    const int n = gemm_configs(kind, &c);
    if (force >= 0 && force < n) return force;
    int best = 0;
    double best_t = 1e300;
    for (int i = 0; i < n; ++i) {
        if (c[i].eff <= 0.f) continue;  // reached only as another entry's deep variant
        const int64_t tiles = ((M + c[i].bm - 1) / c[i].bm) * ((N + c[i].bn - 1) / c[i].bn) * batch;
        const int64_t slots = (int64_t)num_cus * c[i].occupancy;
        const int64_t rounds = (tiles + slots - 1) / slots;
        if (c[i].one_round && rounds > 1) continue;
        const int64_t per_cu = std::min<int64_t>(c[i].occupancy, (tiles + num_cus - 1) / num_cus);
        const double t = (double)rounds * (double)per_cu * c[i].bm * c[i].bn / c[i].eff;
        if (t < best_t * 0.999) {
            best_t = t;
            best = i;
        }
    }
    return best;
}

bool aligned16(const void* p) { return (((uintptr_t)p) & 15) == 0; }

}  // namespace

namespace ingot {

int fail(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(e == hipErrorOutOfMemory ? INGOT_ENOMEM : INGOT_EDEVICE, "%s: %s", what, hipGetErrorString(e));
}

int session_enter(ingot_rocm_session* s) {
    if (!s) return fail(INGOT_EINVAL, "nil session");
    hipError_t e = hipSetDevice(s->device);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    return INGOT_OK;
}

int ws_reserve(ingot_rocm_session* s, size_t bytes, void** out) {
    if (bytes > s->ws_bytes) {
        hipError_t e = hipStreamSynchronize(s->stream);
        if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
        if (s->ws) (void)hipFree(s->ws);
        s->ws = nullptr;
        s->ws_bytes = 0;
        const size_t nb = (size_t)round_up((int64_t)std::max(bytes, (size_t)1 << 21), (int64_t)1 << 21);
        e = hipMalloc(&s->ws, nb);
        if (e != hipSuccess) return hip_fail(e, "workspace hipMalloc");
        s->ws_bytes = nb;
    }
    *out = s->ws;
    return INGOT_OK;
}

// The workspace of one call: the session's growable buffer, or with noalloc
// the device's fixed scratch array (no allocation; sizes beyond it fail).
int call_ws(ingot_rocm_session* s, bool noalloc, size_t bytes, void** out) {
    if (!noalloc) return ws_reserve(s, bytes, out);
    if (bytes > kNoAllocScratchBytes)
        return fail(INGOT_EINVAL, "gemm_noalloc: the call needs %zu bytes of scratch; the fixed maximum is %zu", bytes,
                    kNoAllocScratchBytes);
    *out = s->scratch;
    return INGOT_OK;
}

void* pool_get(ingot_rocm_session* s, size_t bytes) {
    size_t cls = 256;
    while (cls < bytes) cls <<= 1;
    auto it = s->free_bufs.find(cls);
    if (it != s->free_bufs.end() && !it->second.empty()) {
        void* p = it->second.back();
        it->second.pop_back();
        return p;
    }
    void* p = nullptr;
    if (hipMalloc(&p, cls) != hipSuccess) return nullptr;
    s->buf_class[p] = cls;
    return p;
}

void pool_put(ingot_rocm_session* s, void* p) {
    auto it = s->buf_class.find(p);
    if (it == s->buf_class.end()) return;
    s->free_bufs[it->second].push_back(p);
}

Epi make_epi(const ingot_rocm_gemm_args* a) {
    Epi e;
    e.alpha = a->alpha;
    e.beta = a->beta;
    e.c = a->d_c;
    e.ldc = a->ldc;
    e.c_mode = (a->d_c && a->beta != 0.f) ? a->c_mode : INGOT_C_NONE;
    e.act = a->act;
    e.act_alpha = a->act_alpha;
    e.act_beta = a->act_beta;
    e.post = a->post;
    e.post_scale = a->post_scale;
    e.post_shift = a->post_shift;
    e.y_bf16 = a->y_dtype == INGOT_DT_BF16;
    return e;
}

int check_epi(const ingot_rocm_gemm_args* a) {
    if (a->act < INGOT_ACT_NONE || a->act > INGOT_ACT_LEAKYRELU) return fail(INGOT_EINVAL, "unknown activation %d", a->act);
    if (a->y_dtype != 0 && a->y_dtype != INGOT_DT_F32 && a->y_dtype != INGOT_DT_BF16)
        return fail(INGOT_EINVAL, "gemm: Y must be f32 or bf16, got dtype %d", a->y_dtype);
    if (a->d_c && a->beta != 0.f) {
        if (a->c_mode < INGOT_C_NONE || a->c_mode > INGOT_C_SCALAR)
            return fail(INGOT_EINVAL, "unknown C broadcast mode %d", a->c_mode);
        if (a->c_mode == INGOT_C_FULL && a->ldc < a->N) return fail(INGOT_EINVAL, "ldc %lld < N %lld", (long long)a->ldc, (long long)a->N);
    }
    return INGOT_OK;
}

}  // namespace ingot

// ======================= C ABI =======================

extern "C" {

const char* ingot_rocm_last_error(void) { return g_err.c_str(); }

const char* ingot_rocm_version(void) { return "ingot-rocm 0.1 (gfx950)"; }

int ingot_rocm_open(int device, ingot_rocm_session** out) {
    if (!out) return fail(INGOT_EINVAL, "nil out");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
    if (device < 0 || device >= n) return fail(INGOT_EINVAL, "device %d out of range (%d devices)", device, n);
    e = hipSetDevice(device);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(INGOT_EDEVICE, "device %d is %s; this library is built for gfx950", device, prop.gcnArchName);
    if (device >= kMaxDevices) return fail(INGOT_EINVAL, "device %d: at most %d devices", device, kMaxDevices);
    {
        // with `device` current: its copy of the no-alloc scratch array and
        // the event that orders the calls using it
        std::lock_guard<std::mutex> g(g_scratch_mu);
        NoAllocDevice& d = g_noalloc[device];
        if (!d.addr) {
            void* p = nullptr;
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
            if (!p) return fail(INGOT_EDEVICE, "hipGetSymbolAddress(scratch) returned no address");
            e = hipEventCreateWithFlags(&d.done, hipEventDisableTiming);
            if (e != hipSuccess) return hip_fail(e, "no-alloc event");
            d.addr = p;
        }
    }
    auto* s = new ingot_rocm_session();
    s->device = device;
    s->num_cus = prop.multiProcessorCount;
    s->scratch = g_noalloc[device].addr;
    auto env_int = [](const char* name, int dflt) {
        const char* v = getenv(name);
        return v && *v ? atoi(v) : dflt;
    };
    s->force_gemm_cfg = env_int("INGOT_GEMM_CFG", -1);
    s->force_gemv_cfg = env_int("INGOT_GEMV_CFG", 0);
    const int rows = env_int("INGOT_I8G_ROWS", 0);
    s->i8g_rows = rows == 1 || rows == 2 || rows == 4 ? rows : 0;
    s->no_gemv = getenv("INGOT_NO_GEMV") != nullptr;
    s->qconv_path = env_int("INGOT_QCONV_PATH", 0);
    e = hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreate(&s->t0);
    if (e == hipSuccess) e = hipEventCreate(&s->t1);
    if (e != hipSuccess) {
        int rc = hip_fail(e, "session set-up");
        ingot_rocm_close(s);
        return rc;
    }
    *out = s;
    return INGOT_OK;
}

int ingot_rocm_close(ingot_rocm_session* s) {
    if (!s) return INGOT_OK;
    (void)hipSetDevice(s->device);
    if (s->stream) (void)hipStreamSynchronize(s->stream);
    if (s->device >= 0 && s->device < kMaxDevices) {
        // its recorded no-alloc call is complete (the stream is drained)
        NoAllocDevice& d = g_noalloc[s->device];
        std::lock_guard<std::mutex> g(d.mu);
        if (d.last == s) d.last = nullptr;
    }
    for (auto* w : s->weights) {
        if (w->data) (void)hipFree(w->data);
        if (w->colsum) (void)hipFree(w->colsum);
        if (w->gscale) (void)hipFree(w->gscale);
        delete w;
    }
    for (auto& kv : s->buf_class) (void)hipFree(kv.first);
    if (s->ws) (void)hipFree(s->ws);
    if (s->t0) (void)hipEventDestroy(s->t0);
    if (s->t1) (void)hipEventDestroy(s->t1);
    if (s->stream) (void)hipStreamDestroy(s->stream);
    delete s;
    return INGOT_OK;
}

int ingot_rocm_sync(ingot_rocm_session* s) {
    int rc = session_enter(s);
    if (rc) return rc;
    hipError_t e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    return INGOT_OK;
}

int ingot_rocm_stream(ingot_rocm_session* s, void** stream) {
    if (!s || !stream) return fail(INGOT_EINVAL, "nil argument");
    *stream = (void*)s->stream;
    return INGOT_OK;
}

int ingot_rocm_device_alloc(ingot_rocm_session* s, size_t bytes, void** d_out) {
    int rc = session_enter(s);
    if (rc) return rc;
    if (!d_out) return fail(INGOT_EINVAL, "nil out");
    hipError_t e = hipMalloc(d_out, bytes ? bytes : 1);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc");
    return INGOT_OK;
}

int ingot_rocm_device_free(ingot_rocm_session* s, void* d_ptr) {
    int rc = session_enter(s);
    if (rc) return rc;
    if (!d_ptr) return INGOT_OK;
    hipError_t e = hipStreamSynchronize(s->stream);
    if (e == hipSuccess) e = hipFree(d_ptr);
    if (e != hipSuccess) return hip_fail(e, "hipFree");
    return INGOT_OK;
}

int ingot_rocm_host_alloc(ingot_rocm_session* s, size_t bytes, void** h_out) {
    int rc = session_enter(s);
    if (rc) return rc;
    if (!h_out) return fail(INGOT_EINVAL, "nil out");
    hipError_t e = hipHostMalloc(h_out, bytes ? bytes : 1, hipHostMallocDefault);
    if (e != hipSuccess) return hip_fail(e, "hipHostMalloc");
    return INGOT_OK;
}

int ingot_rocm_host_free(ingot_rocm_session* s, void* h_ptr) {
    int rc = session_enter(s);
    if (rc) return rc;
    if (!h_ptr) return INGOT_OK;
    hipError_t e = hipStreamSynchronize(s->stream);
    if (e == hipSuccess) e = hipHostFree(h_ptr);
    if (e != hipSuccess) return hip_fail(e, "hipHostFree");
    return INGOT_OK;
}

static int copy_sync(ingot_rocm_session* s, void* dst, const void* src, size_t bytes, hipMemcpyKind kind) {
    int rc = session_enter(s);
    if (rc) return rc;
    if (!bytes) return INGOT_OK;
    if (!dst || !src) return fail(INGOT_EINVAL, "nil pointer");
    hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, s->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpy");
    return INGOT_OK;
}

int ingot_rocm_memcpy_h2d(ingot_rocm_session* s, void* d_dst, const void* h_src, size_t bytes) {
    return copy_sync(s, d_dst, h_src, bytes, hipMemcpyHostToDevice);
}
int ingot_rocm_memcpy_d2h(ingot_rocm_session* s, void* h_dst, const void* d_src, size_t bytes) {
    return copy_sync(s, h_dst, d_src, bytes, hipMemcpyDeviceToHost);
}
int ingot_rocm_memcpy_d2d(ingot_rocm_session* s, void* d_dst, const void* d_src, size_t bytes) {
    return copy_sync(s, d_dst, d_src, bytes, hipMemcpyDeviceToDevice);
}

int ingot_rocm_memset(ingot_rocm_session* s, void* d_dst, int value, size_t bytes) {
    int rc = session_enter(s);
    if (rc) return rc;
    if (!bytes) return INGOT_OK;
    if (!d_dst) return fail(INGOT_EINVAL, "nil pointer");
    hipError_t e = launch_fill(d_dst, value, bytes, s->stream);
    if (e != hipSuccess) return hip_fail(e, "fill");
    return INGOT_OK;
}

int ingot_rocm_timer_start(ingot_rocm_session* s) {
    int rc = session_enter(s);
    if (rc) return rc;
    hipError_t e = hipEventRecord(s->t0, s->stream);
    if (e != hipSuccess) return hip_fail(e, "hipEventRecord");
    return INGOT_OK;
}

int ingot_rocm_timer_stop(ingot_rocm_session* s, float* ms) {
    int rc = session_enter(s);
    if (rc) return rc;
    if (!ms) return fail(INGOT_EINVAL, "nil out");
    hipError_t e = hipEventRecord(s->t1, s->stream);
    if (e == hipSuccess) e = hipEventSynchronize(s->t1);
    if (e == hipSuccess) e = hipEventElapsedTime(ms, s->t0, s->t1);
    if (e != hipSuccess) return hip_fail(e, "timer");
    return INGOT_OK;
}

// ---------------- weights ----------------

static int weight_pack(ingot_rocm_session* s, int src_dtype, int pack_dtype, int64_t rows, int64_t cols, int64_t ld,
                       int trans, const void* src, bool host, ingot_rocm_weight** out) {
    int rc = session_enter(s);
    if (rc) return rc;
    if (!out) return fail(INGOT_EINVAL, "nil out");
    *out = nullptr;
    if (rows < 1 || cols < 1 || ld < cols || !src)
        return fail(INGOT_EINVAL, "weight: need rows, cols >= 1, ld >= cols and data (rows=%lld cols=%lld ld=%lld)",
                    (long long)rows, (long long)cols, (long long)ld);
    GemmKind kind;
    if (pack_dtype == INGOT_DT_F32 && src_dtype == INGOT_DT_F32) kind = KIND_F32;
    else if (pack_dtype == INGOT_DT_BF16 && (src_dtype == INGOT_DT_F32 || src_dtype == INGOT_DT_BF16)) kind = KIND_BF16;
    else if (pack_dtype == INGOT_DT_I8 && src_dtype == INGOT_DT_I8) kind = KIND_I8;
    else if (pack_dtype == INGOT_PACK_I8G && (src_dtype == INGOT_DT_F32 || src_dtype == INGOT_DT_BF16)) kind = KIND_I8G;
    else return fail(INGOT_EINVAL, "weight: cannot pack dtype %d as %d", src_dtype, pack_dtype);
    const int64_t n = trans ? rows : cols, k = trans ? cols : rows;
    if (n > (int64_t)1 << 30 || k > (int64_t)1 << 30) return fail(INGOT_EINVAL, "weight too large");
    if (kind == KIND_I8G && k % 64 != 0)
        return fail(INGOT_EINVAL, "weight: I8G quantisation needs K a multiple of the group size (64), got %lld",
                    (long long)k);
    auto* w = new ingot_rocm_weight();
    w->pack_dtype = pack_dtype;
    w->kind = kind;
    w->n = n;
    w->k = k;
    w->np = round_up(n, 256);
    w->kp = round_up(k, 256);
    // One extra 128-byte line per row keeps rows off a power-of-two stride.
    w->ldk = w->kp + 128 / kind_size(kind);
    const int esz = elem_size(src_dtype);
    const size_t src_bytes = (size_t)((rows - 1) * ld + cols) * esz;
    const void* dsrc = src;
    void* tmp = nullptr;
    hipError_t e = hipMalloc(&w->data, (size_t)(w->np * w->ldk) * kind_size(kind));
    if (e == hipSuccess && kind == KIND_I8) e = hipMalloc((void**)&w->colsum, sizeof(int32_t) * w->np);
    if (e == hipSuccess && kind == KIND_I8G) e = hipMalloc((void**)&w->gscale, sizeof(float) * w->np * (w->kp / 64));
    if (e == hipSuccess && host) {
        e = hipMalloc(&tmp, src_bytes);
        if (e == hipSuccess) e = hipMemcpyAsync(tmp, src, src_bytes, hipMemcpyHostToDevice, s->stream);
        dsrc = tmp;
    }
    if (e == hipSuccess && kind == KIND_I8G)
        e = launch_quantize_i8g(dsrc, src_dtype, ld, trans, n, k, (int8_t*)w->data, w->gscale, w->np, w->kp, w->ldk,
                                s->stream);
    else if (e == hipSuccess)
        e = launch_pack_weight(dsrc, src_dtype, ld, trans, n, k, w->data, kind, w->np, w->kp, w->ldk, s->stream);
    if (e == hipSuccess && kind == KIND_I8) e = launch_colsum_i8((const int8_t*)w->data, w->kp, w->ldk, w->np, w->colsum, s->stream);
    if (host && e == hipSuccess) e = hipStreamSynchronize(s->stream);
    if (tmp) (void)hipFree(tmp);
    if (e != hipSuccess) {
        if (w->data) (void)hipFree(w->data);
        if (w->colsum) (void)hipFree(w->colsum);
        if (w->gscale) (void)hipFree(w->gscale);
        delete w;
        return hip_fail(e, "weight pack");
    }
    s->weights.push_back(w);
    *out = w;
    return INGOT_OK;
}

int ingot_rocm_weight_upload(ingot_rocm_session* s, int src_dtype, int pack_dtype, int64_t rows, int64_t cols,
                             int64_t ld, int trans, const void* h_src, ingot_rocm_weight** out) {
    return weight_pack(s, src_dtype, pack_dtype, rows, cols, ld, trans, h_src, true, out);
}

int ingot_rocm_weight_pack_device(ingot_rocm_session* s, int src_dtype, int pack_dtype, int64_t rows, int64_t cols,
                                  int64_t ld, int trans, const void* d_src, ingot_rocm_weight** out) {
    return weight_pack(s, src_dtype, pack_dtype, rows, cols, ld, trans, d_src, false, out);
}

int ingot_rocm_weight_free(ingot_rocm_session* s, ingot_rocm_weight* w) {
    int rc = session_enter(s);
    if (rc) return rc;
    if (!w) return INGOT_OK;
    auto it = std::find(s->weights.begin(), s->weights.end(), w);
    if (it == s->weights.end()) return fail(INGOT_EINVAL, "weight does not belong to this session");
    s->weights.erase(it);
    (void)hipStreamSynchronize(s->stream);
    if (w->data) (void)hipFree(w->data);
    if (w->colsum) (void)hipFree(w->colsum);
    if (w->gscale) (void)hipFree(w->gscale);
    delete w;
    return INGOT_OK;
}

int ingot_rocm_weight_info(const ingot_rocm_weight* w, int64_t* n, int64_t* k, int* pack_dtype) {
    if (!w) return fail(INGOT_EINVAL, "nil weight");
    if (n) *n = w->n;
    if (k) *k = w->k;
    if (pack_dtype) *pack_dtype = w->pack_dtype;
    return INGOT_OK;
}

// ---------------- GEMM / GEMV ----------------

static int run_gemv(ingot_rocm_session* s, const ingot_rocm_gemm_args* a, const ingot_rocm_weight* w,
                    bool noalloc = false) {
    GemvArgs g;
    memset(&g, 0, sizeof g);
    g.x = (const float*)a->d_a;
    g.ldx = a->lda;
    g.M = (int)a->M;
    g.K = (int)a->K;
    g.x_vec = aligned16(a->d_a) && (a->lda % 4) == 0;
    g.w = (const uint16_t*)w->data;
    g.ldw = w->ldk;
    g.kp = w->kp;
    g.N = (int)a->N;
    g.split = a->math == INGOT_MATH_BF16 ? 0 : 1;
    g.epi = make_epi(a);
    g.y = a->d_y;
    g.ldy = a->ldy;
    g.cus = s->num_cus;
    const int cfg = s->force_gemv_cfg;
    const bool dma = (cfg == 0 || gemv_cfg_is_dma(cfg)) && gemv_dma_fits(g.M, g.K, g.kp, g.N, g.ldw, g.ldx);
    if (a->M > 4 && !dma) {
        // the MFMA kernel reads x as fragment-ordered bf16 planes (hi, lo)
        void* ws;
        int rc = call_ws(s, noalloc, (size_t)((g.split ? 2 : 1) * 16 * w->kp * 2), &ws);
        if (rc) return rc;
        hipError_t e = launch_pack_x((const float*)a->d_a, a->lda, (int)a->M, (int)a->K, w->kp, g.split,
                                     (uint16_t*)ws, s->stream);
        if (e != hipSuccess) return hip_fail(e, "gemv pack x");
        g.xb = (const uint16_t*)ws;
        g.xb_plane = 16 * w->kp;
    }
    hipError_t e = cfg == 0 && gemv_plain_ok(g) ? launch_gemv_plain(g, s->stream) : launch_gemv_bf16(g, cfg, s->stream);
    if (e != hipSuccess) return hip_fail(e, "gemv launch");
    return INGOT_OK;
}

// Grouped-int8 GEMV: x split once per call into the workspace, then one
// launch per 4 activation rows.
static int run_gemv_i8g(ingot_rocm_session* s, const ingot_rocm_gemm_args* a, const ingot_rocm_weight* w,
                        bool noalloc) {
    const int64_t kp = w->kp, gk = kp / 64;
    if (gk * 4 * 4 * (int64_t)sizeof(float) > 64 * 1024)
        return fail(INGOT_EDECLINED, "gemm: I8G GEMV supports K up to 65536");
    void* ws;
    const size_t plane = (size_t)(a->M * kp);
    int rc = call_ws(s, noalloc, 2 * plane + (size_t)(a->M * gk) * sizeof(float) + 256, &ws);
    if (rc) return rc;
    int8_t* xh = (int8_t*)ws;
    int8_t* xl = xh + plane;
    float* sx = (float*)(((uintptr_t)(xl + plane) + 255) & ~(uintptr_t)255);
    hipError_t e = launch_quantize_x16((const float*)a->d_a, a->lda, (int)a->M, a->K, kp, xh, xl, sx, s->stream);
    if (e != hipSuccess) return hip_fail(e, "quantize x");
    for (int64_t m0 = 0; m0 < a->M; m0 += 4) {
        I8gArgs g;
        memset(&g, 0, sizeof g);
        g.q = (const int8_t*)w->data;
        g.sw = w->gscale;
        g.ldk = w->ldk;
        g.kp = kp;
        g.N = (int)a->N;
        g.M = (int)std::min<int64_t>(4, a->M - m0);
        g.xh = xh + m0 * kp;
        g.xl = xl + m0 * kp;
        g.sx = sx + m0 * gk;
        g.epi = make_epi(a);
        if (g.epi.c_mode == INGOT_C_FULL) g.epi.c += m0 * g.epi.ldc;
        if (g.epi.c_mode == INGOT_C_COL) g.epi.c += m0;
        g.y = (char*)a->d_y + m0 * a->ldy * (g.epi.y_bf16 ? 2 : 4);
        g.ldy = a->ldy;
        const int cfg = s->i8g_rows;
        e = launch_gemv_i8g(g, cfg, s->stream);
        if (e != hipSuccess) return hip_fail(e, "i8g gemv launch");
    }
    return INGOT_OK;
}

static int validate_gemm(ingot_rocm_session* s, const ingot_rocm_gemm_args* a, const ingot_rocm_weight* w) {
    int rc = session_enter(s);
    if (rc) return rc;
    if (!a || !w) return fail(INGOT_EINVAL, "gemm: nil arguments or weight");
    if (a->M < 0 || a->N != w->n || a->K != w->k)
        return fail(INGOT_EINVAL, "gemm: shape M=%lld N=%lld K=%lld does not match weight [%lld,%lld]", (long long)a->M,
                    (long long)a->N, (long long)a->K, (long long)w->n, (long long)w->k);
    if (w->kind == KIND_I8) return fail(INGOT_EINVAL, "gemm: int8 weights run through ingot_rocm_matmul_integer");
    if (w->kind == KIND_I8G && (a->a_dtype != INGOT_DT_F32 || a->trans_a || a->M > 16 || a->batch > 1))
        return fail(INGOT_EDECLINED, "gemm: an int8 (I8G) weight serves decode GEMV only: M <= 16 rows of f32 A");
    if (a->a_dtype != INGOT_DT_F32 && a->a_dtype != INGOT_DT_BF16) return fail(INGOT_EINVAL, "gemm: A must be f32 or bf16");
    if (a->M > 0 && (!a->d_a || !a->d_y)) return fail(INGOT_EINVAL, "gemm: nil A or Y");
    const int64_t amin = a->trans_a ? a->M : a->K;
    if (a->lda < amin) return fail(INGOT_EINVAL, "gemm: lda %lld < %lld", (long long)a->lda, (long long)amin);
    if (a->ldy < a->N) return fail(INGOT_EINVAL, "gemm: ldy %lld < N %lld", (long long)a->ldy, (long long)a->N);
    if (a->M > INT32_MAX / 2 || a->N > INT32_MAX / 2) return fail(INGOT_EINVAL, "gemm: dimension too large");
    if (a->batch > 65535) return fail(INGOT_EINVAL, "gemm: batch %lld > 65535", (long long)a->batch);
    if (a->math == INGOT_MATH_F32 && w->kind != KIND_F32)
        return fail(INGOT_EDECLINED, "gemm: f32 math needs an f32-packed weight");
    if (a->math == INGOT_MATH_BF16 && w->kind != KIND_BF16)
        return fail(INGOT_EDECLINED, "gemm: bf16 math needs a bf16-packed weight");
    if (w->kind == KIND_F32 && a->a_dtype == INGOT_DT_BF16)
        return fail(INGOT_EDECLINED, "gemm: bf16 activations need a bf16-packed weight");
    return check_epi(a);
}

int ingot_rocm_gemv_bf16(ingot_rocm_session* s, const ingot_rocm_gemm_args* a) {
    int rc = validate_gemm(s, a, a ? a->w : nullptr);
    if (rc) return rc;
    if (a->w->kind != KIND_BF16 || a->M > 16 || a->a_dtype != INGOT_DT_F32 || a->trans_a || a->batch > 1)
        return fail(INGOT_EINVAL, "gemv_bf16: needs M <= 16 rows of f32 A (no transA, no batch) and a bf16 weight");
    if (a->M == 0) return INGOT_OK;
    return run_gemv(s, a, a->w);
}

// The GEMM after validation. w may be a session weight or a per-call packed
// operand; stride_b_bytes advances it per batch item (0: shared).
static int run_gemv_i8g(ingot_rocm_session* s, const ingot_rocm_gemm_args* a, const ingot_rocm_weight* w,
                        bool noalloc);

static int gemm_core(ingot_rocm_session* s, const ingot_rocm_gemm_args* a, const ingot_rocm_weight* w,
                     int64_t stride_b_bytes, bool noalloc = false) {
    int rc;
    const int64_t batch = std::max<int64_t>(1, a->batch);
    if (a->M == 0 || a->N == 0) return INGOT_OK;
    if (w->kind == KIND_I8G) return run_gemv_i8g(s, a, w, noalloc);
    // Decode rows take the GEMV: all of M <= 4, and M = 5..16 for N < 4096. At
    // M = 5..16 the wider products run faster as a GEMM of four-stage 32×32
    // tiles (on MI355X at K = 2048, M = 8 and 16: N = 6144 10.7 vs 12.7 µs, N =
    // 11264 13.1 vs 16.2 µs; N = 2048 the GEMV stays ahead, 8.7 vs 10.4 µs).
    if (w->kind == KIND_BF16 && a->M <= 16 && (a->M <= 4 || a->N < 4096) && !a->trans_a &&
        a->a_dtype == INGOT_DT_F32 && batch == 1 && !s->no_gemv)
        return run_gemv(s, a, w, noalloc);

    // bf16 weights with f32 activations: two bf16 planes (f32-class accuracy)
    // unless the caller asked for single bf16 rounding (INGOT_MATH_BF16).
    GemmKind kind = w->kind;
    if (kind == KIND_BF16 && a->a_dtype == INGOT_DT_F32 && a->math != INGOT_MATH_BF16) kind = KIND_BF16X2;
    const int esz = kind_size(kind);
    const int planes = kind == KIND_BF16X2 ? 2 : 1;
    const int64_t kl = round_up(a->K, ktile_elems(kind));
    const int a_esz = elem_size(a->a_dtype);
    const bool a_native = (kind == KIND_BF16 && a->a_dtype == INGOT_DT_BF16) ||
                          (kind == KIND_F32 && a->a_dtype == INGOT_DT_F32);
    const bool direct = a_native && !a->trans_a && a->K % ktile_elems(kind) == 0 && (a->lda * a_esz) % 16 == 0 &&
                        aligned16(a->d_a) && (batch == 1 || (a->stride_a * a_esz) % 16 == 0);
    GemmArgs g;
    memset(&g, 0, sizeof g);
    // Every GEMM operand is addressed with 32-bit buffer offsets.
    // Row offsets of a whole tile past the last row (256 rows) must stay below
    // 2^31 too: the kernel marks past-the-end k-tiles by adding 2^31.
    const int64_t b_extent = w->np * w->ldk * esz;
    const int64_t a_pitch = direct ? a->lda * a_esz : kl * esz;
    const int64_t a_extent = direct ? (a->M - 1) * a_pitch + kl * esz : (int64_t)planes * a->M * kl * esz;
    if (b_extent + 256 * w->ldk * esz >= ((int64_t)1 << 31) || a_extent + 256 * a_pitch >= ((int64_t)1 << 31))
        return fail(INGOT_EDECLINED, "gemm: operand larger than 2 GiB");
    g.a_bytes = (uint32_t)a_extent;
    g.b_bytes = (uint32_t)b_extent;
    if (direct) {
        g.a = (const char*)a->d_a;
        g.lda_bytes = a->lda * a_esz;
        g.stride_a_bytes = a->stride_a * a_esz;
    } else {
        void* ws;
        const int64_t plane = a->M * kl;
        rc = call_ws(s, noalloc, (size_t)(batch * planes * plane * esz), &ws);
        if (rc) return rc;
        hipError_t e = launch_pack_a(a->d_a, a->a_dtype, a->lda, a->trans_a, a->M, a->K, a->stride_a, ws, kind, kl,
                                     planes * plane, (int)batch, s->stream);
        if (e != hipSuccess) return hip_fail(e, "pack A");
        g.a = (const char*)ws;
        g.lda_bytes = kl * esz;
        g.stride_a_bytes = planes * plane * esz;
        g.a_plane_bytes = plane * esz;
    }
    g.b = (const char*)w->data;
    g.ldb_bytes = w->ldk * esz;
    g.stride_b_bytes = stride_b_bytes;
    g.M = (int)a->M;
    g.N = (int)a->N;
    g.kt = (int)(kl * esz / KTILE_BYTES);
    g.b_rows = (int)w->np;
    g.stride_y = a->stride_y;
    g.y = a->d_y;
    g.ldy = a->ldy;
    g.epi = make_epi(a);
    int cfg = pick_config(kind, a->M, a->N, batch, s->num_cus, s->force_gemm_cfg);
    const GemmConfig* c;
    gemm_configs(kind, &c);
    // Operands larger than half the Infinity Cache (256 MB on MI355X) do not
    // stay cached between uses: the product's own output and its neighbours'
    // evict them, so they come from HBM, where the tile whose loads are issued
    // two k-tiles ahead is faster (the configuration tables give the figures).
    if (s->force_gemm_cfg < 0 && c[cfg].deep >= 0 && batch * a_extent + b_extent > kCacheResidentBytes)
        cfg = c[cfg].deep;
    g.tiles_m = (int)((a->M + c[cfg].bm - 1) / c[cfg].bm);
    g.tiles_n = (int)((a->N + c[cfg].bn - 1) / c[cfg].bn);
    hipError_t e = launch_gemm(kind, cfg, g, (int)batch, s->stream);
    if (e != hipSuccess) return hip_fail(e, "gemm launch");
    return INGOT_OK;
}

int ingot_rocm_gemm(ingot_rocm_session* s, const ingot_rocm_gemm_args* a) {
    int rc = validate_gemm(s, a, a ? a->w : nullptr);
    if (rc) return rc;
    return gemm_core(s, a, a->w, 0);
}

int ingot_rocm_gemm_noalloc(ingot_rocm_session* s, const ingot_rocm_gemm_args* a) {
    int rc = validate_gemm(s, a, a ? a->w : nullptr);
    if (rc) return rc;
    NoAllocDevice& d = g_noalloc[s->device];
    std::lock_guard<std::mutex> g(d.mu);
    // Under stream capture the graph's own order applies (an event recorded
    // outside the capture cannot be waited on inside it).
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(s->stream, &cap);
    if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
    const bool order = cap == hipStreamCaptureStatusNone;
    if (order && d.last && d.last != s) {
        e = hipStreamWaitEvent(s->stream, d.done, 0);
        if (e != hipSuccess) return hip_fail(e, "hipStreamWaitEvent");
    }
    rc = gemm_core(s, a, a->w, 0, true);
    if (order) {
        // recorded after a failed call too: a kernel it enqueued before failing
        // may still use the array
        e = hipEventRecord(d.done, s->stream);
        if (e != hipSuccess) return rc ? rc : hip_fail(e, "hipEventRecord");
        d.last = s;
    }
    return rc;
}

int ingot_rocm_session_workspace(const ingot_rocm_session* s, size_t* bytes) {
    if (!s || !bytes) return fail(INGOT_EINVAL, "nil argument");
    *bytes = s->ws_bytes;
    return INGOT_OK;
}

int ingot_rocm_gemm_dynamic_b(ingot_rocm_session* s, const ingot_rocm_gemm_args* a, const void* d_b, int32_t b_dtype,
                              int32_t trans_b, int64_t ldb, int64_t stride_b) {
    int rc = session_enter(s);
    if (rc) return rc;
    if (!a) return fail(INGOT_EINVAL, "gemm_dynamic_b: nil arguments");
    if (a->w) return fail(INGOT_EINVAL, "gemm_dynamic_b: B comes from d_b; the weight handle must be NULL");
    if (b_dtype != INGOT_DT_F32 && b_dtype != INGOT_DT_BF16)
        return fail(INGOT_EINVAL, "gemm_dynamic_b: B must be f32 or bf16");
    if (a->M < 0 || a->N < 0 || a->K < 0 || stride_b < 0)
        return fail(INGOT_EINVAL, "gemm_dynamic_b: negative size or stride");
    if (a->N > 0 && a->K > 0 && ldb < (trans_b ? a->K : a->N))
        return fail(INGOT_EINVAL, "gemm_dynamic_b: ldb %lld < %lld", (long long)ldb, (long long)(trans_b ? a->K : a->N));
    if (a->M == 0 || a->N == 0) return INGOT_OK;
    if (a->K == 0) return fail(INGOT_EDECLINED, "gemm_dynamic_b: K = 0");
    if (!d_b) return fail(INGOT_EINVAL, "gemm_dynamic_b: nil B");
    // f32 B packs as f32 (exact) unless bf16 math was asked for; bf16 B packs
    // as bf16 unless f32 math was asked for (exact widening).
    const bool f32 = a->math == INGOT_MATH_F32 || (b_dtype == INGOT_DT_F32 && a->math != INGOT_MATH_BF16);
    ingot_rocm_weight wt;
    memset(&wt, 0, sizeof wt);
    wt.kind = f32 ? KIND_F32 : KIND_BF16;
    wt.pack_dtype = f32 ? INGOT_DT_F32 : INGOT_DT_BF16;
    wt.n = a->N;
    wt.k = a->K;
    wt.np = round_up(a->N, 256);
    wt.kp = round_up(a->K, 256);
    wt.ldk = wt.kp + 128 / kind_size(wt.kind);
    const int64_t batch = std::max<int64_t>(1, a->batch);
    const int items = stride_b ? (int)batch : 1;
    const int64_t item = wt.np * wt.ldk;
    rc = validate_gemm(s, a, &wt);
    if (rc) return rc;
    wt.data = pool_get(s, (size_t)(items * item * kind_size(wt.kind)));
    if (!wt.data) return fail(INGOT_ENOMEM, "gemm_dynamic_b: cannot allocate the packed B");
    hipError_t e = launch_pack_weight(d_b, b_dtype, ldb, trans_b ? 1 : 0, a->N, a->K, wt.data, wt.kind, wt.np, wt.kp,
                                      wt.ldk, s->stream, items, stride_b, item);
    if (e != hipSuccess) {
        pool_put(s, wt.data);
        return hip_fail(e, "pack B");
    }
    rc = gemm_core(s, a, &wt, stride_b ? item * kind_size(wt.kind) : 0);
    pool_put(s, wt.data);  // stream-ordered: later users of the buffer queue behind this GEMM
    return rc;
}

// The int8 GEMM with its outputs: int32 (yi), dequantised f32 (yf) and/or
// requantised u8/s8 (yq).
static int qgemm(ingot_rocm_session* s, int64_t M, int64_t N, int64_t K, const void* d_a, int32_t a_dtype, int64_t lda,
                 int32_t za, const ingot_rocm_weight* w, int32_t* d_y_i32, const float* d_dq_scale, int64_t n_scale,
                 int32_t dq_zp, float* d_y_f32, void* d_yq, int yq_u8, float rq_mult, float rq_zy) {
    int rc = session_enter(s);
    if (rc) return rc;
    if (!w || w->kind != KIND_I8) return fail(INGOT_EINVAL, "matmul_integer: weight must be packed as int8");
    if (N != w->n || K != w->k || M < 0)
        return fail(INGOT_EINVAL, "matmul_integer: shape M=%lld N=%lld K=%lld does not match weight [%lld,%lld]",
                    (long long)M, (long long)N, (long long)K, (long long)w->n, (long long)w->k);
    if (a_dtype != INGOT_DT_U8 && a_dtype != INGOT_DT_I8) return fail(INGOT_EINVAL, "matmul_integer: A must be u8 or s8");
    if (!d_y_i32 && !d_y_f32 && !d_yq) return fail(INGOT_EINVAL, "matmul_integer: no output");
    if (d_y_f32 && (!d_dq_scale || (n_scale != 1 && n_scale != N)))
        return fail(INGOT_EINVAL, "matmul_integer: dequant scale must have 1 or N elements");
    if (lda < K) return fail(INGOT_EINVAL, "matmul_integer: lda < K");
    if (M == 0) return INGOT_OK;
    if (!d_a) return fail(INGOT_EINVAL, "matmul_integer: nil A");
    const bool u8 = a_dtype == INGOT_DT_U8;
    const int32_t za_s8 = u8 ? za - 128 : za;
    const int64_t kl = round_up(K, 128);
    const bool direct = K % 128 == 0 && lda % 16 == 0 && aligned16(d_a);
    GemmArgs g;
    memset(&g, 0, sizeof g);
    const int64_t a_pitch = direct ? lda : kl;
    const int64_t a_extent = direct ? (M - 1) * lda + kl : M * kl;
    if ((w->np + 256) * w->ldk >= ((int64_t)1 << 31) || a_extent + 256 * a_pitch >= ((int64_t)1 << 31))
        return fail(INGOT_EDECLINED, "matmul_integer: operand larger than 2 GiB");
    g.a_bytes = (uint32_t)a_extent;
    g.b_bytes = (uint32_t)(w->np * w->ldk);
    if (direct) {
        g.a = (const char*)d_a;
        g.lda_bytes = lda;
        g.a_xor = u8 ? 1 : 0;
    } else {
        void* ws;
        rc = ws_reserve(s, (size_t)(M * kl), &ws);
        if (rc) return rc;
        hipError_t e = launch_pack_a(d_a, a_dtype, lda, 0, M, K, 0, ws, KIND_I8, kl, 0, 1, s->stream);
        if (e != hipSuccess) return hip_fail(e, "pack A");
        g.a = (const char*)ws;
        g.lda_bytes = kl;
    }
    g.b = (const char*)w->data;
    g.ldb_bytes = w->ldk;
    g.M = (int)M;
    g.N = (int)N;
    g.kt = (int)(kl / KTILE_BYTES);
    g.b_rows = (int)w->np;
    g.ldy = N;
    g.qepi.colsum = w->colsum;
    g.qepi.neg_za = (int32_t)(0u - (uint32_t)za_s8);
    g.qepi.yi = d_y_i32;
    g.qepi.yf = d_y_f32;
    g.qepi.scale = d_dq_scale;
    g.qepi.n_scale = n_scale;
    g.qepi.dq_zp = dq_zp;
    g.qepi.yq = d_yq;
    g.qepi.yq_u8 = yq_u8;
    g.qepi.rq_mult = rq_mult;
    g.qepi.rq_zy = rq_zy;
    const int cfg = pick_config(KIND_I8, M, N, 1, s->num_cus, s->force_gemm_cfg);
    const GemmConfig* c;
    gemm_configs(KIND_I8, &c);
    g.tiles_m = (int)((M + c[cfg].bm - 1) / c[cfg].bm);
    g.tiles_n = (int)((N + c[cfg].bn - 1) / c[cfg].bn);
    hipError_t e = launch_gemm(KIND_I8, cfg, g, 1, s->stream);
    if (e != hipSuccess) return hip_fail(e, "qgemm launch");
    return INGOT_OK;
}

int ingot_rocm_matmul_integer(ingot_rocm_session* s, int64_t M, int64_t N, int64_t K, const void* d_a, int32_t a_dtype,
                              int64_t lda, int32_t za, const ingot_rocm_weight* w, int32_t* d_y_i32,
                              const float* d_dq_scale, int64_t n_scale, int32_t dq_zp, float* d_y_f32) {
    return qgemm(s, M, N, K, d_a, a_dtype, lda, za, w, d_y_i32, d_dq_scale, n_scale, dq_zp, d_y_f32, nullptr, 0, 0.f,
                 0.f);
}

int ingot_rocm_qlinear_matmul(ingot_rocm_session* s, int64_t M, int64_t N, int64_t K, const void* d_a, int32_t a_dtype,
                              int64_t lda, int32_t za, const ingot_rocm_weight* w, float mult, int32_t zy,
                              int32_t y_dtype, void* d_y) {
    if (y_dtype != INGOT_DT_U8 && y_dtype != INGOT_DT_I8)
        return fail(INGOT_EINVAL, "qlinear_matmul: output must be u8 or s8");
    if (!d_y && M > 0 && N > 0) return fail(INGOT_EINVAL, "qlinear_matmul: nil Y");
    return qgemm(s, M, N, K, d_a, a_dtype, lda, za, w, nullptr, nullptr, 1, 0, nullptr, d_y,
                 y_dtype == INGOT_DT_U8 ? 1 : 0, mult, (float)zy);
}

// convOut (ops/conv.go:110-113); C++ division truncates toward zero as Go's does.
static int64_t conv_out(int64_t in, int64_t k, int64_t stride, int64_t dil, int64_t pa, int64_t pb) {
    return (in + pa + pb - (dil * (k - 1) + 1)) / stride + 1;
}

int ingot_rocm_qlinear_conv(ingot_rocm_session* s, const ingot_rocm_qconv_args* a, const ingot_rocm_weight* w) {
    int rc = session_enter(s);
    if (rc) return rc;
    if (!a) return fail(INGOT_EINVAL, "qlinear_conv: nil args");
    if (!w || w->kind != KIND_I8) return fail(INGOT_EINVAL, "qlinear_conv: weight must be packed as int8");
    if (a->x_dtype != INGOT_DT_U8 && a->x_dtype != INGOT_DT_I8)
        return fail(INGOT_EINVAL, "qlinear_conv: x must be u8 or s8");
    if (a->y_dtype != INGOT_DT_U8 && a->y_dtype != INGOT_DT_I8)
        return fail(INGOT_EINVAL, "qlinear_conv: output must be u8 or s8");
    if (a->n < 0 || a->c < 1 || a->h < 1 || a->w < 1 || a->m < 1 || a->kh < 1 || a->kw < 1 || a->group < 1)
        return fail(INGOT_EINVAL, "qlinear_conv: bad dims");
    if (a->c % a->group != 0 || a->m % a->group != 0) return fail(INGOT_EINVAL, "qlinear_conv: channel mismatch");
    if (a->stride_h < 1 || a->stride_w < 1 || a->dilation_h < 1 || a->dilation_w < 1 || a->pad_top < 0 ||
        a->pad_left < 0 || a->pad_bottom < 0 || a->pad_right < 0)
        return fail(INGOT_EINVAL, "qlinear_conv: strides and dilations must be >= 1, pads >= 0");
    const int64_t Cg = a->c / a->group, Mg = a->m / a->group, K = Cg * a->kh * a->kw;
    if (w->n != a->m || w->k != K)
        return fail(INGOT_EINVAL, "qlinear_conv: weight [%lld,%lld] does not match M=%lld K=%lld", (long long)w->n,
                    (long long)w->k, (long long)a->m, (long long)K);
    const int64_t OH = conv_out(a->h, a->kh, a->stride_h, a->dilation_h, a->pad_top, a->pad_bottom);
    const int64_t OW = conv_out(a->w, a->kw, a->stride_w, a->dilation_w, a->pad_left, a->pad_right);
    if (OH < 0 || OW < 0) return fail(INGOT_EINVAL, "qlinear_conv: negative output size %lldx%lld", (long long)OH,
                                      (long long)OW);
    const bool u8 = a->x_dtype == INGOT_DT_U8;
    if (u8 ? (a->zx < 0 || a->zx > 255) : (a->zx < -128 || a->zx > 127))
        return fail(INGOT_EDECLINED, "qlinear_conv: x zero point %d outside the range of x", a->zx);
    const int64_t P = OH * OW, total = a->n * a->m * P;
    const int64_t lim = (int64_t)1 << 31;
    if (a->n * a->c * a->h * a->w >= lim || total >= lim || a->h * a->w >= lim / 8 || a->group > 65535)
        return fail(INGOT_EDECLINED, "qlinear_conv: tensor larger than 2 GiB");
    if (total == 0) return INGOT_OK;
    if (!a->d_x || !a->d_mult || !a->d_y) return fail(INGOT_EINVAL, "qlinear_conv: nil x, mult or y");
    QconvGeom g;
    g.N = (int)a->n, g.C = (int)a->c, g.H = (int)a->h, g.W = (int)a->w, g.M = (int)a->m, g.G = (int)a->group;
    g.Cg = (int)Cg, g.KH = (int)a->kh, g.KW = (int)a->kw, g.sh = (int)a->stride_h, g.sw = (int)a->stride_w;
    g.dh = (int)a->dilation_h, g.dw = (int)a->dilation_w, g.pt = (int)a->pad_top, g.pl = (int)a->pad_left;
    g.OH = (int)OH, g.OW = (int)OW;
    const int yu8 = a->y_dtype == INGOT_DT_U8 ? 1 : 0;
    // Route: a GEMM needs output-channel and reduction width to fill MFMA
    // tiles; depthwise and narrow groups run direct. INGOT_QCONV_PATH=1/2
    // forces direct/GEMM (tests run both routes on the same cases).
    const int path = s->qconv_path;
    const int64_t kgl = round_up(K, 128);
    const bool gemm = path == 2 || (path != 1 && Mg >= 16 && K >= 32);
    if (!gemm) {
        hipError_t e = launch_qconv_direct(a->d_x, u8 ? 1 : 0, g, (const int8_t*)w->data, w->ldk, a->d_bias,
                                           a->d_mult, a->zx, (float)a->zy, yu8, a->d_y, s->stream);
        if (e != hipSuccess) return hip_fail(e, "qconv direct");
        return INGOT_OK;
    }
    // Images per chunk: the column matrix of one chunk stays under ~512 MiB
    // and each group's rows under the 2 GiB buffer-offset limit.
    const int64_t per_img = P * kgl;
    if ((P + 256) * kgl >= lim || (w->np + 256) * w->ldk >= lim)
        return fail(INGOT_EDECLINED, "qlinear_conv: column matrix or weight larger than 2 GiB");
    int64_t ipc = std::max<int64_t>(1, ((int64_t)512 << 20) / (a->group * per_img));
    ipc = std::min(ipc, std::max<int64_t>(1, (lim - 256 * kgl) / per_img - 1));
    ipc = std::min(ipc, a->n);
    void* ws;
    rc = ws_reserve(s, (size_t)(a->group * ipc * per_img), &ws);
    if (rc) return rc;
    const int cfg0 = pick_config(KIND_I8, ipc * P, Mg, a->group, s->num_cus, s->force_gemm_cfg);
    const GemmConfig* cf;
    gemm_configs(KIND_I8, &cf);
    for (int64_t n0 = 0; n0 < a->n; n0 += ipc) {
        const int64_t imgs = std::min(ipc, a->n - n0);
        const int64_t rows = imgs * P;
        const int64_t col_group = rows * kgl;
        hipError_t e = launch_qim2col((const uint8_t*)a->d_x + n0 * a->c * a->h * a->w, g, (int)rows, (int)K,
                                      (int)kgl, (uint8_t)a->zx, ws, col_group, s->stream);
        if (e != hipSuccess) return hip_fail(e, "qim2col");
        GemmArgs ga;
        memset(&ga, 0, sizeof ga);
        ga.a = (const char*)ws;
        ga.lda_bytes = kgl;
        ga.stride_a_bytes = col_group;
        ga.a_bytes = (uint32_t)col_group;
        ga.a_xor = u8 ? 1 : 0;
        ga.b = (const char*)w->data;
        ga.ldb_bytes = w->ldk;
        ga.stride_b_bytes = a->group > 1 ? Mg * w->ldk : 0;
        ga.b_bytes = (uint32_t)(a->group > 1 ? Mg * w->ldk : w->np * w->ldk);
        ga.b_rows = (int)w->np;
        ga.M = (int)rows;
        ga.N = (int)Mg;
        ga.kt = (int)(kgl / KTILE_BYTES);
        ga.stride_y = Mg * P;
        ga.ldy = Mg;
        ga.qepi.colsum = w->colsum;
        ga.qepi.neg_za = (int32_t)(0u - (uint32_t)(u8 ? a->zx - 128 : a->zx));
        ga.qepi.yq = (uint8_t*)a->d_y + n0 * a->m * P;
        ga.qepi.yq_u8 = yu8;
        ga.qepi.rq_zy = (float)a->zy;
        ga.qepi.rq_mults = a->d_mult;
        ga.qepi.bias = a->d_bias;
        ga.qepi.col_batch = (int32_t)Mg;
        ga.qepi.conv_p = (int32_t)P;
        ga.qepi.conv_img = a->m * P;
        const int cfg = rows == ipc * P ? cfg0 : pick_config(KIND_I8, rows, Mg, a->group, s->num_cus, s->force_gemm_cfg);
        ga.tiles_m = (int)((rows + cf[cfg].bm - 1) / cf[cfg].bm);
        ga.tiles_n = (int)((Mg + cf[cfg].bn - 1) / cf[cfg].bn);
        e = launch_gemm(KIND_I8, cfg, ga, (int)a->group, s->stream);
        if (e != hipSuccess) return hip_fail(e, "qconv gemm");
    }
    return INGOT_OK;
}

int ingot_rocm_dequantize_linear(ingot_rocm_session* s, const void* d_x, int32_t x_dtype, int64_t n,
                                 const float* d_scale, int64_t n_scale, int64_t inner, const void* d_zp,
                                 int32_t zp_dtype, int64_t n_zp, float* d_y) {
    int rc = session_enter(s);
    if (rc) return rc;
    if (x_dtype != INGOT_DT_U8 && x_dtype != INGOT_DT_I8 && x_dtype != INGOT_DT_I32)
        return fail(INGOT_EINVAL, "dequantize_linear: unsupported input dtype %d", x_dtype);
    if (d_zp && zp_dtype != INGOT_DT_U8 && zp_dtype != INGOT_DT_I8 && zp_dtype != INGOT_DT_I32)
        return fail(INGOT_EINVAL, "dequantize_linear: unsupported zero_point dtype %d", zp_dtype);
    if (n_scale < 1 || (d_zp && n_zp != 1 && n_zp != n_scale))
        return fail(INGOT_EINVAL, "dequantize_linear: scale/zero_point sizes %lld/%lld", (long long)n_scale, (long long)n_zp);
    if (n == 0) return INGOT_OK;
    if (!d_x || !d_scale || !d_y) return fail(INGOT_EINVAL, "dequantize_linear: nil pointer");
    hipError_t e = launch_dequant(d_x, x_dtype, n, d_scale, n_scale, inner, d_zp, zp_dtype, n_zp, d_y, s->stream);
    if (e != hipSuccess) return hip_fail(e, "dequant launch");
    return INGOT_OK;
}

int ingot_rocm_activation(ingot_rocm_session* s, const float* d_x, float* d_y, int64_t rows, int64_t cols,
                          const float* d_bias, int32_t act, float act_alpha, float act_beta, int32_t post,
                          float post_scale, float post_shift) {
    int rc = session_enter(s);
    if (rc) return rc;
    if (act < INGOT_ACT_NONE || act > INGOT_ACT_LEAKYRELU) return fail(INGOT_EINVAL, "unknown activation %d", act);
    if (rows < 0 || cols < 0) return fail(INGOT_EINVAL, "negative size");
    if (rows * cols == 0) return INGOT_OK;
    if (!d_x || !d_y) return fail(INGOT_EINVAL, "nil pointer");
    hipError_t e = launch_activation(d_x, d_y, rows, cols, d_bias, act, act_alpha, act_beta, post, post_scale,
                                     post_shift, s->stream);
    if (e != hipSuccess) return hip_fail(e, "activation launch");
    return INGOT_OK;
}

int ingot_rocm_cast_bf16(ingot_rocm_session* s, const float* d_x, uint16_t* d_y, int64_t n) {
    int rc = session_enter(s);
    if (rc) return rc;
    if (n == 0) return INGOT_OK;
    if (!d_x || !d_y || n < 0) return fail(INGOT_EINVAL, "cast_bf16: bad arguments");
    hipError_t e = launch_cast_bf16(d_x, d_y, n, s->stream);
    if (e != hipSuccess) return hip_fail(e, "cast launch");
    return INGOT_OK;
}

}  // extern "C"
