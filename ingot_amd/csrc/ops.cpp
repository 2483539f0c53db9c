// Operator layer: ONNX-semantics ops over device tensors, mirroring the
// reference's op plugin interface (ops/op.go:96-181): a registry of builders
// keyed by (domain, op, since-opset), NodeInfo with typed attributes, Op.Run
// that validates, allocates outputs from the session pool (ctx.NewUninit)
// and dispatches to the gfx950 kernels. Error texts follow the reference ops
// so a caller sees the same failures (NodeInfo.Errorf: "Op(name): msg").
//
// Ops: Gemm@7 and MatMul@1 (ops/matmul.go:27-139, 305-438, 454-472),
// MatMulInteger@10 and QLinearMatMul@10 (ops/quant.go:791-928, 942-943), QLinearConv@10
// (ops/quant.go:323-420, 941), DequantizeLinear@10
// (ops/quant.go:168-230, 947-949), and the activation nodes a GEMM epilogue
// can absorb: Relu@6, Sigmoid@6, HardSwish@14, LeakyRelu@6, HardSigmoid@6,
// Gelu@20, ingot.Gelu@1, ingot.SiLU@1 (ops/elementwise.go:486-545).

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "runtime.hpp"

namespace ingot {
namespace ops {

// ---------------- attributes, NodeInfo ----------------

struct Attr {
    char kind = 0;  // 'i', 'f', 's', 'I' (int list)
    int64_t i = 0;
    float f = 0;
    std::string s;
    std::vector<int64_t> ints;
};

struct Attrs {
    std::map<std::string, Attr> m;
    bool has(const std::string& k) const { return m.count(k) != 0; }
    int64_t Int(const std::string& k, int64_t def) const {
        auto it = m.find(k);
        return it != m.end() && it->second.kind == 'i' ? it->second.i : def;
    }
    float Float(const std::string& k, float def) const {
        auto it = m.find(k);
        if (it == m.end()) return def;
        if (it->second.kind == 'f') return it->second.f;
        if (it->second.kind == 'i') return (float)it->second.i;
        return def;
    }
    std::string String(const std::string& k, const std::string& def) const {
        auto it = m.find(k);
        return it != m.end() && it->second.kind == 's' ? it->second.s : def;
    }
    std::vector<int64_t> Ints(const std::string& k, const std::vector<int64_t>& def) const {
        auto it = m.find(k);
        return it != m.end() && it->second.kind == 'I' ? it->second.ints : def;
    }
};

// Parses "i:transB=1;f:alpha=0.5;s:ingot_act=gelu;I:strides=2,2".
int parse_attrs(const char* text, Attrs* out) {
    if (!text) return INGOT_OK;
    std::string t(text);
    size_t pos = 0;
    while (pos < t.size()) {
        size_t end = t.find(';', pos);
        if (end == std::string::npos) end = t.size();
        std::string item = t.substr(pos, end - pos);
        pos = end + 1;
        if (item.empty()) continue;
        if (item.size() < 4 || item[1] != ':' || item.find('=') == std::string::npos)
            return fail(INGOT_EINVAL, "bad attribute %s (want kind:name=value)", item.c_str());
        const size_t eq = item.find('=');
        Attr a;
        a.kind = item[0];
        const std::string name = item.substr(2, eq - 2);
        const std::string val = item.substr(eq + 1);
        char* ep = nullptr;
        switch (a.kind) {
            case 'i': a.i = strtoll(val.c_str(), &ep, 10); break;
            case 'f': a.f = strtof(val.c_str(), &ep); break;
            case 's': a.s = val; ep = nullptr; break;
            case 'I': {
                ep = nullptr;
                size_t q = 0;
                while (q < val.size()) {
                    size_t c = val.find(',', q);
                    if (c == std::string::npos) c = val.size();
                    const std::string v = val.substr(q, c - q);
                    char* e2 = nullptr;
                    const long long x = strtoll(v.c_str(), &e2, 10);
                    if (v.empty() || (e2 && *e2)) return fail(INGOT_EINVAL, "bad attribute value %s", item.c_str());
                    a.ints.push_back(x);
                    q = c + 1;
                }
                break;
            }
            default: return fail(INGOT_EINVAL, "bad attribute kind %c", a.kind);
        }
        if (ep && *ep) return fail(INGOT_EINVAL, "bad attribute value %s", item.c_str());
        out->m[name] = a;
    }
    return INGOT_OK;
}

const char* dtype_name(int dt) {
    switch (dt) {
        case INGOT_DT_F32: return "f32";
        case INGOT_DT_F16: return "f16";
        case INGOT_DT_BF16: return "bf16";
        case INGOT_DT_I8: return "i8";
        case INGOT_DT_U8: return "u8";
        case INGOT_DT_I16: return "i16";
        case INGOT_DT_I32: return "i32";
        case INGOT_DT_I64: return "i64";
        case INGOT_DT_BOOL: return "bool";
    }
    return "invalid";
}

int dtype_size(int dt) {
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

typedef std::vector<int64_t> Shape;

std::string shape_str(const Shape& s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); ++i) {
        if (i) r += " ";
        r += std::to_string(s[i]);
    }
    return r + "]";
}

int64_t numel(const Shape& s) {
    int64_t n = 1;
    for (auto d : s) n *= d;
    return n;
}

struct NodeInfo {
    std::string name, op_type, domain;
    int version = 0;
    Attrs attrs;
    // NodeInfo.Errorf (ops/op.go:179-181)
    int errorf(int code, const char* fmt, ...) const __attribute__((format(printf, 3, 4))) {
        char buf[768];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        return fail(code, "%s(%s): %s", op_type.c_str(), name.c_str(), buf);
    }
};

// A tensor as an op sees it (nil data = omitted optional input).
struct T {
    int dtype = 0;
    Shape shape;
    void* data = nullptr;
    bool present() const { return data != nullptr || (dtype != 0 && numel(shape) == 0); }
    int rank() const { return (int)shape.size(); }
    int64_t dim(int i) const { return shape[i]; }
    int64_t n() const { return numel(shape); }
    std::string str() const { return std::string(dtype_name(dtype)) + shape_str(shape); }
};

struct Ctx {
    ingot_rocm_session* s;
    std::vector<ingot_rocm_tensor>* outs;
    // ctx.NewUninit (ops/op.go:86-93): pooled device storage
    int new_uninit(int dt, const Shape& sh, T* out) {
        if (sh.size() > 8) return fail(INGOT_EINVAL, "rank %zu > 8", sh.size());
        out->dtype = dt;
        out->shape = sh;
        const size_t bytes = (size_t)numel(sh) * dtype_size(dt);
        out->data = pool_get(s, bytes ? bytes : 1);
        if (!out->data) return fail(INGOT_ENOMEM, "pool allocation of %zu bytes failed", bytes);
        return INGOT_OK;
    }
    // ctx.Out
    void emit(const T& t) {
        ingot_rocm_tensor o;
        memset(&o, 0, sizeof o);
        o.dtype = t.dtype;
        o.rank = t.rank();
        for (int i = 0; i < o.rank; ++i) o.dims[i] = t.shape[i];
        o.data = t.data;
        outs->push_back(o);
    }
};

class Op {
   public:
    virtual ~Op() {}
    virtual int run(Ctx& ctx, const std::vector<T>& in) = 0;
    // A graph plan (graph.cpp): the activation the product's store applies,
    // bf16 products against constant weights (GPUBF16), a bf16 output.
    // Only matrix products take one.
    virtual int plan(int fused_act, bool half, bool out_bf16) {
        (void)fused_act, (void)half, (void)out_bf16;
        return INGOT_EDECLINED;
    }
    // Inputs the caller declared constant (graph constants: their device
    // storage holds the same values on every run). Only those are packed
    // once and cached; every other operand is packed per call, since a
    // pooled device buffer is handed back at the same address with new
    // contents (the reference's GPU session likewise caches only graph
    // constants, by value id: bf16Const, graph/gpuops_darwin_arm64.go:610-629).
    std::vector<char> const_in;
    bool is_const(size_t i) const { return i < const_in.size() && const_in[i]; }
};

typedef std::function<int(const NodeInfo&, std::unique_ptr<Op>*)> Builder;

struct Entry {
    int since;
    Builder build;
};

std::mutex& reg_mu() {
    static std::mutex m;
    return m;
}
std::map<std::pair<std::string, std::string>, std::vector<Entry>>& registry() {
    static std::map<std::pair<std::string, std::string>, std::vector<Entry>> r;
    return r;
}

// Register (ops/op.go:132-141): entries sorted by since ascending.
void Register(const std::string& domain, const std::string& op, int since, Builder b) {
    std::lock_guard<std::mutex> g(reg_mu());
    auto& es = registry()[{domain, op}];
    es.push_back({since, b});
    std::sort(es.begin(), es.end(), [](const Entry& a, const Entry& b) { return a.since < b.since; });
}

// Lookup (ops/op.go:143-160): the newest builder with since <= version.
int Lookup(const std::string& domain, const std::string& op, int version, Builder* out) {
    std::lock_guard<std::mutex> g(reg_mu());
    auto it = registry().find({domain, op});
    if (it == registry().end() || it->second.empty())
        return fail(INGOT_EINVAL, "ops: unsupported op \"%s\" (domain \"%s\")", op.c_str(), domain.c_str());
    const Entry* best = nullptr;
    for (auto& e : it->second)
        if (e.since <= version) best = &e;
    if (!best)
        return fail(INGOT_EINVAL, "ops: op \"%s\" (domain \"%s\") not supported at opset %d (have since %d)", op.c_str(),
                    domain.c_str(), version, it->second[0].since);
    *out = best->build;
    return INGOT_OK;
}

// ---------------- device helpers ----------------

int read_ints(ingot_rocm_session* s, const T& t, std::vector<int32_t>* out) {
    const int64_t n = t.n();
    out->resize(n);
    if (!n) return INGOT_OK;
    std::vector<uint8_t> raw((size_t)n * dtype_size(t.dtype));
    int rc = ingot_rocm_memcpy_d2h(s, raw.data(), t.data, raw.size());
    if (rc) return rc;
    for (int64_t i = 0; i < n; ++i) {
        switch (t.dtype) {
            case INGOT_DT_U8: (*out)[i] = raw[i]; break;
            case INGOT_DT_I8: (*out)[i] = (int8_t)raw[i]; break;
            case INGOT_DT_I32: {
                int32_t v;
                memcpy(&v, &raw[i * 4], 4);
                (*out)[i] = v;
                break;
            }
            default: return fail(INGOT_EINVAL, "not an integer tensor");
        }
    }
    return INGOT_OK;
}

// First element of an f32 tensor (per-tensor quantisation scales).
int read_f32_first(ingot_rocm_session* s, const T& t, float* out) {
    if (t.dtype != INGOT_DT_F32 || t.n() < 1) return fail(INGOT_EINVAL, "scale must be a non-empty f32 tensor");
    return ingot_rocm_memcpy_d2h(s, out, t.data, sizeof(float));
}

// bCache (ops/matmul.go:200-236): the packed form of a B that is the same
// storage every run; a B whose storage ever changes marks the op dynamic and
// is packed per call.
struct BCache {
    std::mutex mu;
    const void* src = nullptr;
    int64_t len = 0;
    int trans = -1, pack_dtype = 0;
    bool dyn = false;
    ingot_rocm_weight* pb = nullptr;

    // Returns the cached pack, or nullptr when the operand is not a declared
    // constant or has proven dynamic (the caller packs per call).
    int get(ingot_rocm_session* s, const T& b, bool constant, int trans_, int pack_dtype_, ingot_rocm_weight** out) {
        std::lock_guard<std::mutex> g(mu);
        *out = nullptr;
        if (!constant || dyn || b.n() == 0) return INGOT_OK;
        if (src == b.data && len == b.n() && trans == trans_ && pack_dtype == pack_dtype_) {
            *out = pb;
            return INGOT_OK;
        }
        if (src != nullptr) {  // storage changed: not a constant
            dyn = true;
            if (pb) ingot_rocm_weight_free(s, pb);
            pb = nullptr;
            src = nullptr;
            return INGOT_OK;
        }
        int rc = ingot_rocm_weight_pack_device(s, b.dtype, pack_dtype_, b.dim(0), b.dim(1), b.dim(1), trans_, b.data, &pb);
        if (rc) return rc;
        src = b.data;
        len = b.n();
        trans = trans_;
        pack_dtype = pack_dtype_;
        *out = pb;
        return INGOT_OK;
    }
    void release(ingot_rocm_session* s) {
        if (pb) ingot_rocm_weight_free(s, pb);
        pb = nullptr;
    }
};

// Per-call pack of a dynamic operand, freed when the call's work is queued.
struct TempWeights {
    ingot_rocm_session* s;
    std::vector<ingot_rocm_weight*> ws;
    explicit TempWeights(ingot_rocm_session* s_) : s(s_) {}
    ~TempWeights() {
        for (auto* w : ws) ingot_rocm_weight_free(s, w);
    }
    int pack(int src_dt, int pack_dt, int64_t rows, int64_t cols, int trans, const void* d, ingot_rocm_weight** out) {
        int rc = ingot_rocm_weight_pack_device(s, src_dt, pack_dt, rows, cols, cols, trans, d, out);
        if (!rc) ws.push_back(*out);
        return rc;
    }
};

ingot_rocm_gemm_args gemm_args() {
    ingot_rocm_gemm_args a;
    memset(&a, 0, sizeof a);
    a.alpha = 1.f;
    a.post_scale = 1.f;
    a.batch = 1;
    return a;
}

// ---------------- Gemm ----------------

// gemmOp (ops/matmul.go:14-139): Y = alpha·op(A)·op(B) + beta·C.
class GemmOp : public Op {
   public:
    NodeInfo n;
    float alpha, beta;
    bool transA, transB;
    // quantI8 (ops/matmul.go:19-23): ingot_weight_quant="int8" runs decode
    // shapes (M <= 4, transB, K % 64 == 0) on an int8 copy of the weight.
    bool quant_i8 = false;
    BCache cache, cache_i8;
    ingot_rocm_session* s;
    int fused_act = INGOT_ACT_NONE;
    bool half = false, out_bf16 = false;
    ~GemmOp() override {
        cache.release(s);
        cache_i8.release(s);
    }
    int plan(int act, bool h, bool ob) override {
        fused_act = act, half = h, out_bf16 = ob;
        return INGOT_OK;
    }

    int run(Ctx& ctx, const std::vector<T>& in) override {
        if (in.size() < 2 || !in[0].present() || !in[1].present()) return n.errorf(INGOT_EINVAL, "need A and B");
        const T& a = in[0];
        const T& b = in[1];
        const bool bf16B = b.dtype == INGOT_DT_BF16 && !transA;
        // a bf16 A is a bf16-resident activation under a half plan
        const bool a_ok = a.dtype == INGOT_DT_F32 || (half && a.dtype == INGOT_DT_BF16 && !transA);
        if (!a_ok || (b.dtype != INGOT_DT_F32 && !bf16B) || a.rank() != 2 || b.rank() != 2)
            return n.errorf(INGOT_EINVAL, "need 2-D f32 A and f32 (or bf16 weight) B, got %s %s", a.str().c_str(),
                            b.str().c_str());
        int64_t M = a.dim(0), K = a.dim(1);
        if (transA) std::swap(M, K);
        int64_t Kb = b.dim(0), N = b.dim(1);
        if (transB) std::swap(Kb, N);
        if (K != Kb) return n.errorf(INGOT_EINVAL, "inner dim mismatch %lld vs %lld", (long long)K, (long long)Kb);
        ingot_rocm_gemm_args g = gemm_args();
        if (in.size() > 2 && in[2].present() && beta != 0) {
            const T& c = in[2];
            if (c.dtype != INGOT_DT_F32) return n.errorf(INGOT_EINVAL, "C must be f32, got %s", c.str().c_str());
            const int64_t cn = c.n();
            if (cn == M * N && (c.rank() == 2 || (c.rank() == 1 && M == 1))) {
                g.c_mode = INGOT_C_FULL;
                g.ldc = N;
            } else if (cn == N) {
                g.c_mode = INGOT_C_ROW;
            } else if (cn == M && c.rank() == 2) {
                g.c_mode = INGOT_C_COL;
            } else if (cn == 1) {
                g.c_mode = INGOT_C_SCALAR;
            } else {
                return n.errorf(INGOT_EINVAL, "cannot broadcast C %s to [%lld,%lld]", shape_str(c.shape).c_str(),
                                (long long)M, (long long)N);
            }
            g.d_c = (const float*)c.data;
            g.beta = beta;
        }
        const int ydt = out_bf16 ? INGOT_DT_BF16 : INGOT_DT_F32;
        T out;
        int rc = ctx.new_uninit(ydt, {M, N}, &out);
        if (rc) return rc;
        if (M > 0 && N > 0) {
            if (K == 0) {
                // empty reduction: Y = beta·C (or 0)
                rc = ingot_rocm_memset(s, out.data, 0, (size_t)(M * N * dtype_size(ydt)));
                if (rc) return rc;
                if (g.c_mode != INGOT_C_NONE) {
                    ingot_rocm_tensor tmp;
                    (void)tmp;
                    return n.errorf(INGOT_EDECLINED, "K = 0 with C is run by the CPU op");
                }
                ctx.emit(out);
                return INGOT_OK;
            }
            // ops/matmul.go:77-86 (the reference takes it where its int8 dot is SIMD)
            const bool i8g = quant_i8 && transB && !transA && M <= 4 && K % 64 == 0 && a.dtype == INGOT_DT_F32;
            const int pack_dt =
                i8g ? INGOT_PACK_I8G : (b.dtype == INGOT_DT_BF16 || half ? INGOT_DT_BF16 : INGOT_DT_F32);
            // the weight source is [N,K] when transB (rows = b.dim(0))
            ingot_rocm_weight* w = nullptr;
            rc = (i8g ? cache_i8 : cache).get(s, b, is_const(1), transB ? 1 : 0, pack_dt, &w);
            if (rc) return rc;
            TempWeights tmp(s);
            if (!w) {
                rc = tmp.pack(b.dtype, pack_dt, b.dim(0), b.dim(1), transB ? 1 : 0, b.data, &w);
                if (rc) return rc;
            }
            g.M = M;
            g.N = N;
            g.K = K;
            g.d_a = a.data;
            g.a_dtype = a.dtype;
            g.trans_a = transA ? 1 : 0;
            g.lda = a.dim(1);
            g.w = w;
            g.alpha = alpha;
            g.act = fused_act;
            if (half && !i8g) g.math = INGOT_MATH_BF16;
            g.d_y = (float*)out.data;
            g.y_dtype = ydt;
            g.ldy = N;
            rc = ingot_rocm_gemm(s, &g);
            if (rc) return n.errorf(rc, "%s", ingot_rocm_last_error());
        }
        ctx.emit(out);
        return INGOT_OK;
    }
};

// ---------------- MatMul ----------------

int broadcast_shape(const Shape& a, const Shape& b, Shape* out) {
    const size_t n = std::max(a.size(), b.size());
    out->assign(n, 0);
    for (size_t i = 0; i < n; ++i) {
        const int64_t ja = (int64_t)a.size() - (int64_t)n + (int64_t)i;
        const int64_t jb = (int64_t)b.size() - (int64_t)n + (int64_t)i;
        const int64_t da = ja >= 0 ? a[ja] : 1, db = jb >= 0 ? b[jb] : 1;
        if (da == db || db == 1) (*out)[i] = da;
        else if (da == 1) (*out)[i] = db;
        else return fail(INGOT_EINVAL, "cannot broadcast %s with %s", shape_str(a).c_str(), shape_str(b).c_str());
    }
    return INGOT_OK;
}

// broadcastStridesIn (ops/broadcast.go:50-68): strides in matrices, 0 on broadcast dims.
std::vector<int64_t> broadcast_strides(const Shape& shape, const Shape& out) {
    std::vector<int64_t> st(out.size(), 0);
    int64_t acc = 1;
    for (int64_t i = (int64_t)shape.size() - 1; i >= 0; --i) {
        const int64_t oi = (int64_t)out.size() - (int64_t)shape.size() + i;
        st[oi] = shape[i] == 1 ? 0 : acc;
        acc *= shape[i];
    }
    return st;
}

// matmulOp (ops/matmul.go:282-438): NumPy matmul with batch broadcasting, an
// optional optimizer-attached bias [N] (graph/fuse_matmul_bias.go) and the
// ingot_act="gelu" activation, both fused into the GEMM store here.
class MatMulOp : public Op {
   public:
    NodeInfo n;
    std::string act;
    BCache cache;
    ingot_rocm_session* s;
    bool bf16_weights = false;
    int fused_act = INGOT_ACT_NONE;
    bool half = false, out_bf16 = false;
    ~MatMulOp() override { cache.release(s); }
    int plan(int act_code, bool h, bool ob) override {
        fused_act = act_code, half = h, out_bf16 = ob;
        return INGOT_OK;
    }

    int run(Ctx& ctx, const std::vector<T>& in) override {
        if (in.size() < 2 || in.size() > 3 || !in[0].present() || !in[1].present())
            return n.errorf(INGOT_EINVAL, "need 2 inputs (+ optional bias)");
        const T& a = in[0];
        const T& b = in[1];
        const float* bias = nullptr;
        if (in.size() == 3 && in[2].present()) {
            if (in[2].dtype != INGOT_DT_F32 || b.rank() == 0 || in[2].n() != b.shape.back())
                return n.errorf(INGOT_EINVAL, "bias must be f32 [N], got %s %s", dtype_name(in[2].dtype),
                                shape_str(in[2].shape).c_str());
            bias = (const float*)in[2].data;
        }
        // a bf16 A is a bf16-resident activation under a half plan
        if ((a.dtype != INGOT_DT_F32 && !(half && a.dtype == INGOT_DT_BF16)) || b.dtype != INGOT_DT_F32)
            return n.errorf(INGOT_EINVAL, "only f32");
        Shape as = a.shape, bs = b.shape;
        if (as.empty() || bs.empty()) return n.errorf(INGOT_EINVAL, "scalar operands not allowed");
        bool squeezeM = false, squeezeN = false;
        if (as.size() == 1) {
            as = {1, as[0]};
            squeezeM = true;
        }
        if (bs.size() == 1) {
            bs = {bs[0], 1};
            squeezeN = true;
        }
        int64_t M = as[as.size() - 2], K = as[as.size() - 1];
        const int64_t Kb = bs[bs.size() - 2], N = bs[bs.size() - 1];
        if (K != Kb)
            return n.errorf(INGOT_EINVAL, "inner dim mismatch: %s · %s", shape_str(a.shape).c_str(),
                            shape_str(b.shape).c_str());
        const Shape batchA(as.begin(), as.end() - 2), batchB(bs.begin(), bs.end() - 2);
        Shape batch;
        int rc = broadcast_shape(batchA, batchB, &batch);
        if (rc) return n.errorf(INGOT_EINVAL, "%s", ingot_rocm_last_error());
        Shape oshape = batch;
        oshape.push_back(M);
        oshape.push_back(N);
        const int ydt = out_bf16 ? INGOT_DT_BF16 : INGOT_DT_F32;
        T out;
        rc = ctx.new_uninit(ydt, oshape, &out);
        if (rc) return rc;
        int64_t nb = numel(batch);
        const int act_code = act == "gelu" ? INGOT_ACT_GELU_ERF : fused_act;
        if (out.n() > 0) {
            if (K == 0) return n.errorf(INGOT_EDECLINED, "K = 0 is run by the CPU op");
            ingot_rocm_gemm_args g = gemm_args();
            g.K = K;
            g.N = N;
            g.a_dtype = a.dtype;
            g.lda = K;
            g.ldy = N;
            g.act = act_code;
            g.y_dtype = ydt;
            if (half) g.math = INGOT_MATH_BF16;
            if (bias) {
                g.d_c = bias;
                g.c_mode = INGOT_C_ROW;
                g.beta = 1.f;
            }
            const int pack_dt = bf16_weights || half ? INGOT_DT_BF16 : INGOT_DT_F32;
            if (!batchB.empty() && (a.dtype != INGOT_DT_F32 || ydt != INGOT_DT_F32))
                return n.errorf(INGOT_EINVAL, "a batched right operand takes f32 operands only");
            if (batchB.empty()) {
                // 2-D rhs shared by every batch: one GEMM over nb·M rows
                // (ops/matmul.go:351-361; on the GPU always, the CPU's size
                // threshold was a scheduling choice).
                M *= nb;
                nb = 1;
                ingot_rocm_weight* w = nullptr;
                Shape b2 = {bs[0], bs[1]};
                T bt = b;
                bt.shape = b2;
                rc = cache.get(s, bt, is_const(1), 0, pack_dt, &w);
                if (rc) return rc;
                TempWeights tmp(s);
                if (!w) {
                    rc = tmp.pack(INGOT_DT_F32, pack_dt, b2[0], b2[1], 0, b.data, &w);
                    if (rc) return rc;
                }
                g.M = M;
                g.d_a = a.data;
                g.w = w;
                g.d_y = (float*)out.data;
                rc = ingot_rocm_gemm(s, &g);
                if (rc) return n.errorf(rc, "%s", ingot_rocm_last_error());
            } else {
                // Batched right operand (attention Q·Kᵀ / P·V): per-batch products
                // with broadcast operand offsets (ops/matmul.go:375-403). B is an
                // activation, packed on the device per call; when both operands'
                // matrix offsets are linear in the output batch index (equal batch
                // shapes, or one side broadcast whole) all items run as one
                // batched launch, otherwise one call per item.
                const auto sa = broadcast_strides(batchA, batch);
                const auto sb = broadcast_strides(batchB, batch);
                std::vector<int64_t> offA((size_t)nb), offB((size_t)nb), idx(batch.size(), 0);
                for (int64_t bi = 0; bi < nb; ++bi) {
                    int64_t oa = 0, ob = 0;
                    for (size_t d = 0; d < idx.size(); ++d) {
                        oa += idx[d] * sa[d];
                        ob += idx[d] * sb[d];
                    }
                    offA[(size_t)bi] = oa;
                    offB[(size_t)bi] = ob;
                    for (int64_t d = (int64_t)idx.size() - 1; d >= 0; --d) {
                        if (++idx[(size_t)d] < batch[(size_t)d]) break;
                        idx[(size_t)d] = 0;
                    }
                }
                const int64_t cA = nb > 1 ? offA[1] - offA[0] : 0, cB = nb > 1 ? offB[1] - offB[0] : 0;
                bool linear = offA[0] == 0 && offB[0] == 0;
                for (int64_t bi = 0; bi < nb && linear; ++bi)
                    linear = offA[(size_t)bi] == bi * cA && offB[(size_t)bi] == bi * cB;
                g.M = M;
                const float* A = (const float*)a.data;
                const float* B = (const float*)b.data;
                float* Y = (float*)out.data;
                if (linear) {
                    for (int64_t b0 = 0; b0 < nb; b0 += 65535) {
                        g.batch = std::min<int64_t>(65535, nb - b0);
                        g.d_a = A + b0 * cA * M * K;
                        g.stride_a = cA * M * K;
                        g.d_y = Y + b0 * M * N;
                        g.stride_y = M * N;
                        rc = ingot_rocm_gemm_dynamic_b(s, &g, B + b0 * cB * K * N, INGOT_DT_F32, 0, N, cB * K * N);
                        if (rc) return n.errorf(rc, "%s", ingot_rocm_last_error());
                    }
                } else {
                    g.batch = 1;
                    for (int64_t bi = 0; bi < nb; ++bi) {
                        g.d_a = A + offA[(size_t)bi] * M * K;
                        g.d_y = Y + bi * M * N;
                        rc = ingot_rocm_gemm_dynamic_b(s, &g, B + offB[(size_t)bi] * K * N, INGOT_DT_F32, 0, N, 0);
                        if (rc) return n.errorf(rc, "%s", ingot_rocm_last_error());
                    }
                }
            }
        }
        if (squeezeM || squeezeN) {
            Shape fs = batch;
            if (!squeezeM) fs.push_back(oshape[oshape.size() - 2]);
            if (!squeezeN) fs.push_back(N);
            out.shape = fs;
        }
        ctx.emit(out);
        return INGOT_OK;
    }
};

// ---------------- MatMulInteger ----------------

// qmatmulOp (ops/quant.go:791-928): MatMulInteger (requant = false, int32
// out) and QLinearMatMul (requant = true, u8/s8 out).
class MatMulIntegerOp : public Op {
   public:
    NodeInfo n;
    bool requant = false;
    ingot_rocm_session* s;
    std::mutex mu;
    const void* pack_src = nullptr;
    int64_t pack_k = -1, pack_n = -1;
    ingot_rocm_weight* packed = nullptr;
    ~MatMulIntegerOp() override {
        if (packed) ingot_rocm_weight_free(s, packed);
    }

    // s8Weights (ops/quant.go:285-302)
    int s8_weights(const T& w, const T* wzp) {
        if (w.dtype != INGOT_DT_I8)
            return n.errorf(INGOT_EINVAL,
                            "only s8 weights supported (got %s); u8 weights are not emitted by standard quantizers",
                            dtype_name(w.dtype));
        if (wzp && wzp->present()) {
            if (wzp->dtype != INGOT_DT_I8)
                return n.errorf(INGOT_EINVAL, "weight zero_point dtype %s unsupported", dtype_name(wzp->dtype));
            std::vector<int32_t> z;
            int rc = read_ints(s, *wzp, &z);
            if (rc) return rc;
            for (auto v : z)
                if (v != 0) return n.errorf(INGOT_EINVAL, "non-zero weight zero_point unsupported (symmetric s8 weights only)");
        }
        return INGOT_OK;
    }

    // bWeights (ops/quant.go:801-829): a declared-constant B is packed once
    // per storage; any other B is packed per call into `tmp`.
    int b_weights(const T& b, bool constant, int64_t k, int64_t nn, TempWeights& tmp, ingot_rocm_weight** out) {
        if (!constant) return tmp.pack(INGOT_DT_I8, INGOT_DT_I8, k, nn, 0, b.data, out);
        std::lock_guard<std::mutex> g(mu);
        if (packed && pack_src == b.data && pack_k == k && pack_n == nn) {
            *out = packed;
            return INGOT_OK;
        }
        if (packed) ingot_rocm_weight_free(s, packed);
        packed = nullptr;
        int rc = ingot_rocm_weight_pack_device(s, INGOT_DT_I8, INGOT_DT_I8, k, nn, nn, 0, b.data, &packed);
        if (rc) return rc;
        pack_src = b.data;
        pack_k = k;
        pack_n = nn;
        *out = packed;
        return INGOT_OK;
    }

    int run(Ctx& ctx, const std::vector<T>& in) override {
        auto opt = [&](size_t i) { return in.size() > i && in[i].present() ? &in[i] : nullptr; };
        const T *pa, *pb, *aZp, *bZp, *aScale = nullptr, *bScale = nullptr, *yScale = nullptr, *yZp = nullptr;
        if (requant) {
            if (in.size() < 8 || !in[0].present() || !in[1].present() || !in[3].present() || !in[4].present() ||
                !in[6].present())
                return n.errorf(INGOT_EINVAL, "need 8 inputs");
            pa = &in[0], aScale = &in[1], aZp = opt(2), pb = &in[3], bScale = &in[4], bZp = opt(5), yScale = &in[6],
            yZp = opt(7);
        } else {
            if (in.size() < 2 || !in[0].present() || !in[1].present()) return n.errorf(INGOT_EINVAL, "need 2-4 inputs");
            pa = &in[0], pb = &in[1], aZp = opt(2), bZp = opt(3);
        }
        const T& a = *pa;
        const T& b = *pb;
        int rc = s8_weights(b, bZp);
        if (rc) return rc;
        if (a.rank() != 2 || b.rank() != 2 || a.dim(1) != b.dim(0))
            return n.errorf(INGOT_EINVAL, "2-D matmul only (a %s, b %s)", shape_str(a.shape).c_str(),
                            shape_str(b.shape).c_str());
        const int64_t m = a.dim(0), k = a.dim(1), nn = b.dim(1);
        int32_t za = 0;
        if (aZp) {
            if (aZp->dtype != INGOT_DT_U8 && aZp->dtype != INGOT_DT_I8 && aZp->dtype != INGOT_DT_I32)
                return n.errorf(INGOT_EINVAL, "per-tensor a zero_point only");
            std::vector<int32_t> z;
            rc = read_ints(s, *aZp, &z);
            if (rc) return rc;
            if (z.size() != 1) return n.errorf(INGOT_EINVAL, "per-tensor a zero_point only");
            za = z[0];
        }
        if (a.dtype != INGOT_DT_U8 && a.dtype != INGOT_DT_I8)
            return n.errorf(INGOT_EINVAL, "activations must be u8 or s8, got %s", dtype_name(a.dtype));
        // QLinearMatMul: per-tensor scales (element 0, ops/quant.go:911) and the
        // output zero point, whose dtype is the output dtype (quantParams,
        // ops/quant.go:50-72; absent: u8, 0)
        float mult = 0.f;
        int32_t zy = 0;
        int ydt = INGOT_DT_I32;
        if (requant) {
            float sa, sb, sy;
            if ((rc = read_f32_first(s, *aScale, &sa)) || (rc = read_f32_first(s, *bScale, &sb)) ||
                (rc = read_f32_first(s, *yScale, &sy)))
                return n.errorf(rc, "%s", ingot_rocm_last_error());
            volatile float ab = sa * sb;
            mult = ab / sy;
            ydt = INGOT_DT_U8;
            if (yZp) {
                std::vector<int32_t> z;
                if (yZp->dtype != INGOT_DT_U8 && yZp->dtype != INGOT_DT_I8)
                    return n.errorf(INGOT_EINVAL, "unsupported output quantization");
                rc = read_ints(s, *yZp, &z);
                if (rc) return rc;
                if (z.size() != 1) return n.errorf(INGOT_EINVAL, "unsupported output quantization");
                ydt = yZp->dtype;
                zy = z[0];
            }
        }
        T out;
        rc = ctx.new_uninit(ydt, {m, nn}, &out);
        if (rc) return rc;
        if (m > 0 && nn > 0) {
            if (k == 0) {
                // empty reduction: every product is 0, so Y = sat(zy) (or 0 for int32 out)
                const int fill = !requant ? 0 : ydt == INGOT_DT_U8 ? std::min(255, std::max(0, zy))
                                                                   : std::min(127, std::max(-128, zy));
                rc = ingot_rocm_memset(s, out.data, fill & 0xFF,
                                       (size_t)(m * nn * (requant ? 1 : 4)));
                if (rc) return rc;
            } else {
                ingot_rocm_weight* w = nullptr;
                TempWeights tmp(s);
                rc = b_weights(b, is_const(requant ? 3 : 1), k, nn, tmp, &w);
                if (rc) return rc;
                if (requant)
                    rc = ingot_rocm_qlinear_matmul(s, m, nn, k, a.data, a.dtype, k, za, w, mult, zy, ydt, out.data);
                else
                    rc = ingot_rocm_matmul_integer(s, m, nn, k, a.data, a.dtype, k, za, w, (int32_t*)out.data,
                                                   nullptr, 1, 0, nullptr);
                if (rc) return n.errorf(rc, "%s", ingot_rocm_last_error());
            }
        }
        ctx.emit(out);
        return INGOT_OK;
    }
};

// ---------------- QLinearConv ----------------

// qlinearConvOp (ops/quant.go:323-420) over the conv geometry of buildConv
// (ops/conv.go:61-108): group, strides, dilations, pads, auto_pad; 1-D
// attributes lift to 2-D (spatial2D, ops/conv.go:86-99). Inputs x, x_scale,
// x_zero_point, w, w_scale, w_zero_point, y_scale, y_zero_point[, B].
class QLinearConvOp : public Op {
   public:
    NodeInfo n;
    ingot_rocm_session* s;
    int64_t group = 1;
    int64_t strides[2] = {1, 1}, dilations[2] = {1, 1}, pads[4] = {0, 0, 0, 0};
    std::string auto_pad;
    bool three_d = false;
    std::mutex mu;
    const void* pack_src = nullptr;
    int64_t pack_m = -1, pack_k = -1;
    ingot_rocm_weight* packed = nullptr;
    ~QLinearConvOp() override {
        if (packed) ingot_rocm_weight_free(s, packed);
    }

    int build() {
        group = n.attrs.Int("group", 1);
        auto_pad = n.attrs.String("auto_pad", "NOTSET");
        auto st = n.attrs.Ints("strides", {1, 1});
        auto di = n.attrs.Ints("dilations", {1, 1});
        auto pa = n.attrs.Ints("pads", {0, 0, 0, 0});
        // isConv3D: three spatial dims (ops/conv.go:64-68) build, then Run rejects
        // the rank-5 input (only 2-D conv)
        auto ks = n.attrs.Ints("kernel_shape", {});
        if (ks.size() == 3 || st.size() == 3 || di.size() == 3 || pa.size() == 6) {
            three_d = true;
            return INGOT_OK;
        }
        if (st.size() == 1) st = {1, st[0]};
        if (di.size() == 1) di = {1, di[0]};
        if (pa.size() == 2) pa = {0, pa[0], 0, pa[1]};
        if (st.size() != 2 || di.size() != 2 || pa.size() != 4) {
            auto js = [](const std::vector<int64_t>& v) {
                std::string r = "[";
                for (size_t i = 0; i < v.size(); ++i) r += (i ? " " : "") + std::to_string(v[i]);
                return r + "]";
            };
            return n.errorf(INGOT_EINVAL, "only 1-D and 2-D conv supported (strides=%s dilations=%s pads=%s)",
                            js(st).c_str(), js(di).c_str(), js(pa).c_str());
        }
        for (int i = 0; i < 2; ++i) strides[i] = st[i], dilations[i] = di[i];
        for (int i = 0; i < 4; ++i) pads[i] = pa[i];
        return INGOT_OK;
    }

    // convOp.resolvePads (ops/conv.go:115-136)
    int resolve_pads(int64_t h, int64_t w, int64_t kh, int64_t kw, int64_t out[4]) {
        for (int i = 0; i < 4; ++i) out[i] = pads[i];
        if (auto_pad == "NOTSET" || auto_pad.empty()) return INGOT_OK;
        if (auto_pad == "VALID") {
            for (int i = 0; i < 4; ++i) out[i] = 0;
            return INGOT_OK;
        }
        if (auto_pad != "SAME_UPPER" && auto_pad != "SAME_LOWER")
            return n.errorf(INGOT_EINVAL, "unsupported auto_pad \"%s\"", auto_pad.c_str());
        const int64_t in[2] = {h, w}, k[2] = {kh, kw};
        for (int d = 0; d < 2; ++d) {
            const int64_t st = strides[d], dl = dilations[d];
            const int64_t o = (in[d] + st - 1) / st;
            const int64_t total = std::max<int64_t>(0, (o - 1) * st + dl * (k[d] - 1) + 1 - in[d]);
            const int64_t a = auto_pad == "SAME_LOWER" ? (total + 1) / 2 : total / 2;
            out[d] = a;
            out[d + 2] = total - a;
        }
        return INGOT_OK;
    }

    // the packed [M, K] weight, once per weight storage (qlinearConvOp.fill, ops/quant.go:753-789)
    int weights(const T& w, int64_t m, int64_t k, ingot_rocm_weight** out) {
        std::lock_guard<std::mutex> g(mu);
        if (packed && pack_src == w.data && pack_m == m && pack_k == k) {
            *out = packed;
            return INGOT_OK;
        }
        if (packed) ingot_rocm_weight_free(s, packed);
        packed = nullptr;
        int rc = ingot_rocm_weight_pack_device(s, INGOT_DT_I8, INGOT_DT_I8, m, k, k, 1, w.data, &packed);
        if (rc) return rc;
        pack_src = w.data, pack_m = m, pack_k = k;
        *out = packed;
        return INGOT_OK;
    }

    // quantParams (ops/quant.go:50-72): one zero point value and the dtype it names
    int zero_point(const T* zp, std::vector<int32_t>* z, int* dt) {
        *dt = INGOT_DT_U8;
        z->assign(1, 0);
        if (!zp) return INGOT_OK;
        *dt = zp->dtype;
        if (zp->dtype != INGOT_DT_U8 && zp->dtype != INGOT_DT_I8 && zp->dtype != INGOT_DT_I32)
            return n.errorf(INGOT_EINVAL, "unsupported quantization parameter dtype");
        return read_ints(s, *zp, z);
    }

    int run(Ctx& ctx, const std::vector<T>& in) override {
        if (in.size() < 8) return n.errorf(INGOT_EINVAL, "need 8-9 inputs");
        auto opt = [&](size_t i) { return in.size() > i && in[i].present() ? &in[i] : nullptr; };
        for (size_t i : {0, 1, 3, 4, 6})
            if (!in[i].present()) return n.errorf(INGOT_EINVAL, "need 8-9 inputs");
        const T &x = in[0], &xScale = in[1], &w = in[3], &wScale = in[4], &yScale = in[6];
        const T *xZp = opt(2), *wZp = opt(5), *yZp = opt(7), *bias = opt(8);
        // s8Weights (ops/quant.go:285-302)
        if (w.dtype != INGOT_DT_I8)
            return n.errorf(INGOT_EINVAL,
                            "only s8 weights supported (got %s); u8 weights are not emitted by standard quantizers",
                            dtype_name(w.dtype));
        int rc;
        if (wZp) {
            if (wZp->dtype != INGOT_DT_I8)
                return n.errorf(INGOT_EINVAL, "weight zero_point dtype %s unsupported", dtype_name(wZp->dtype));
            std::vector<int32_t> z;
            if ((rc = read_ints(s, *wZp, &z))) return rc;
            for (auto v : z)
                if (v != 0)
                    return n.errorf(INGOT_EINVAL, "non-zero weight zero_point unsupported (symmetric s8 weights only)");
        }
        std::vector<int32_t> xz, yz;
        int xdt, ydt;
        if ((rc = zero_point(xZp, &xz, &xdt)) || (rc = zero_point(yZp, &yz, &ydt))) return rc;
        if (xz.size() != 1 || yz.size() != 1 || ydt == INGOT_DT_I32)
            return n.errorf(INGOT_EINVAL, "per-tensor activation/output quantization only");
        if (three_d || x.rank() != 4 || w.rank() != 4) return n.errorf(INGOT_EINVAL, "only 2-D conv");
        const int64_t N = x.dim(0), C = x.dim(1), H = x.dim(2), W = x.dim(3);
        const int64_t M = w.dim(0), Cg = w.dim(1), KH = w.dim(2), KW = w.dim(3);
        if (group < 1 || C != Cg * group || M % group != 0) return n.errorf(INGOT_EINVAL, "channel mismatch");
        if (x.dtype != INGOT_DT_U8 && x.dtype != INGOT_DT_I8)
            return n.errorf(INGOT_EINVAL, "activations must be u8 or s8, got %s", dtype_name(x.dtype));
        if (ydt != INGOT_DT_U8 && ydt != INGOT_DT_I8)
            return n.errorf(INGOT_EINVAL, "per-tensor activation/output quantization only");
        int64_t pd[4];
        if ((rc = resolve_pads(H, W, KH, KW, pd))) return rc;
        const int64_t OH = (H + pd[0] + pd[2] - (dilations[0] * (KH - 1) + 1)) / strides[0] + 1;
        const int64_t OW = (W + pd[1] + pd[3] - (dilations[1] * (KW - 1) + 1)) / strides[1] + 1;
        if (OH < 0 || OW < 0) return n.errorf(INGOT_EINVAL, "negative output size %lldx%lld", (long long)OH, (long long)OW);
        if (bias && (bias->dtype != INGOT_DT_I32 || bias->n() != M))
            return n.errorf(INGOT_EINVAL, "bias must be int32 [%lld], got %s", (long long)M, bias->str().c_str());
        if (wScale.n() != 1 && wScale.n() != M)
            return n.errorf(INGOT_EINVAL, "w_scale must have 1 or %lld elements", (long long)M);
        // requant multipliers x_scale·w_scale[m]/y_scale, each product and
        // quotient rounded to f32 (ops/quant.go:380-390)
        float xs, ys;
        if ((rc = read_f32_first(s, xScale, &xs)) || (rc = read_f32_first(s, yScale, &ys)))
            return n.errorf(rc, "%s", ingot_rocm_last_error());
        if (wScale.dtype != INGOT_DT_F32) return n.errorf(INGOT_EINVAL, "w_scale must be f32");
        std::vector<float> wsc((size_t)wScale.n()), mult((size_t)M);
        if ((rc = ingot_rocm_memcpy_d2h(s, wsc.data(), wScale.data, wsc.size() * sizeof(float))))
            return n.errorf(rc, "%s", ingot_rocm_last_error());
        for (int64_t m = 0; m < M; ++m) {
            volatile float t = xs * wsc[wsc.size() > 1 ? m : 0];
            mult[m] = t / ys;
        }
        T out;
        if ((rc = ctx.new_uninit(ydt, {N, M, OH, OW}, &out))) return rc;
        if (N * M * OH * OW > 0) {
            ingot_rocm_weight* pw = nullptr;
            if ((rc = weights(w, M, Cg * KH * KW, &pw))) return n.errorf(rc, "%s", ingot_rocm_last_error());
            void* dm = pool_get(s, (size_t)M * sizeof(float));
            if (!dm) return n.errorf(INGOT_ENOMEM, "pool allocation failed");
            if ((rc = ingot_rocm_memcpy_h2d(s, dm, mult.data(), (size_t)M * sizeof(float)))) {
                pool_put(s, dm);
                return n.errorf(rc, "%s", ingot_rocm_last_error());
            }
            ingot_rocm_qconv_args a;
            memset(&a, 0, sizeof a);
            a.n = N, a.c = C, a.h = H, a.w = W, a.m = M, a.kh = KH, a.kw = KW, a.group = group;
            a.stride_h = strides[0], a.stride_w = strides[1], a.dilation_h = dilations[0], a.dilation_w = dilations[1];
            a.pad_top = pd[0], a.pad_left = pd[1], a.pad_bottom = pd[2], a.pad_right = pd[3];
            a.d_x = x.data, a.x_dtype = x.dtype, a.zx = xz[0];
            a.d_mult = (const float*)dm;
            a.d_bias = bias ? (const int32_t*)bias->data : nullptr;
            a.zy = yz[0], a.y_dtype = ydt, a.d_y = out.data;
            rc = ingot_rocm_qlinear_conv(s, &a, pw);
            pool_put(s, dm);  // stream-ordered: a later user queues behind this conv
            if (rc) return n.errorf(rc, "%s", ingot_rocm_last_error());
        }
        ctx.emit(out);
        return INGOT_OK;
    }
};

// ---------------- DequantizeLinear ----------------

// dequantizeLinearOp (ops/quant.go:168-230).
class DequantizeLinearOp : public Op {
   public:
    NodeInfo n;
    int64_t axis;
    ingot_rocm_session* s;

    int run(Ctx& ctx, const std::vector<T>& in) override {
        if (in.size() < 2 || !in[0].present() || !in[1].present()) return n.errorf(INGOT_EINVAL, "need x and scale");
        const T& x = in[0];
        const T& sc = in[1];
        const T* zp = in.size() > 2 && in[2].present() ? &in[2] : nullptr;
        if (sc.dtype != INGOT_DT_F32) return n.errorf(INGOT_EINVAL, "scale must be f32");
        if (zp && zp->dtype != INGOT_DT_U8 && zp->dtype != INGOT_DT_I8 && zp->dtype != INGOT_DT_I32)
            return n.errorf(INGOT_EINVAL, "unsupported zero_point dtype");
        if (x.dtype != INGOT_DT_U8 && x.dtype != INGOT_DT_I8 && x.dtype != INGOT_DT_I32)
            return n.errorf(INGOT_EINVAL, "unsupported input dtype %s", dtype_name(x.dtype));
        const int64_t nsc = sc.n();
        const int64_t nzp = zp ? zp->n() : 1;
        T out;
        int rc = ctx.new_uninit(INGOT_DT_F32, x.shape, &out);
        if (rc) return rc;
        int64_t inner = 1;
        if (nsc != 1) {
            const int64_t r = x.rank();
            int64_t ax = axis < 0 ? axis + r : axis;
            if (ax < 0 || ax >= r || x.shape[ax] != nsc)
                return n.errorf(INGOT_EINVAL, "per-axis scale len %lld vs dims %s axis %lld", (long long)nsc,
                                shape_str(x.shape).c_str(), (long long)axis);
            for (int64_t d = ax + 1; d < r; ++d) inner *= x.shape[d];
            if (nzp != 1 && nzp != nsc) return n.errorf(INGOT_EINVAL, "zero_point len %lld vs scale len %lld", (long long)nzp, (long long)nsc);
        }
        // per-tensor: z = zpi[0] (ops/quant.go:192-194)
        rc = ingot_rocm_dequantize_linear(s, x.data, x.dtype, x.n(), (const float*)sc.data, nsc, inner,
                                          zp ? zp->data : nullptr, zp ? zp->dtype : 0, nsc == 1 ? 1 : nzp,
                                          (float*)out.data);
        if (rc) return n.errorf(rc, "%s", ingot_rocm_last_error());
        ctx.emit(out);
        return INGOT_OK;
    }
};

// ---------------- activation nodes ----------------

class UnaryOp : public Op {
   public:
    NodeInfo n;
    int act;
    float a = 0, b = 0;
    ingot_rocm_session* s;
    int run(Ctx& ctx, const std::vector<T>& in) override {
        if (in.empty() || !in[0].present()) return n.errorf(INGOT_EINVAL, "need an input");
        const T& x = in[0];
        if (x.dtype != INGOT_DT_F32) return n.errorf(INGOT_EINVAL, "only f32");
        T out;
        int rc = ctx.new_uninit(INGOT_DT_F32, x.shape, &out);
        if (rc) return rc;
        rc = ingot_rocm_activation(s, (const float*)x.data, (float*)out.data, 1, x.n(), nullptr, act, a, b, 0, 1.f, 0.f);
        if (rc) return n.errorf(rc, "%s", ingot_rocm_last_error());
        ctx.emit(out);
        return INGOT_OK;
    }
};

// Builders need the session; it is bound at op creation.
thread_local ingot_rocm_session* t_build_session = nullptr;

void register_all() {
    static std::once_flag once;
    std::call_once(once, [] {
        // ops/matmul.go:454-472
        Register("", "Gemm", 7, [](const NodeInfo& n, std::unique_ptr<Op>* out) {
            auto op = std::make_unique<GemmOp>();
            op->n = n;
            op->alpha = n.attrs.Float("alpha", 1);
            op->beta = n.attrs.Float("beta", 1);
            op->transA = n.attrs.Int("transA", 0) != 0;
            op->transB = n.attrs.Int("transB", 0) != 0;
            op->quant_i8 = n.attrs.String("ingot_weight_quant", "") == "int8";
            op->s = t_build_session;
            *out = std::move(op);
            return INGOT_OK;
        });
        Register("", "MatMul", 1, [](const NodeInfo& n, std::unique_ptr<Op>* out) {
            const std::string act = n.attrs.String("ingot_act", "");
            if (!act.empty() && act != "gelu") return n.errorf(INGOT_EINVAL, "unknown ingot_act \"%s\"", act.c_str());
            auto op = std::make_unique<MatMulOp>();
            op->n = n;
            op->act = act;
            op->s = t_build_session;
            op->bf16_weights = n.attrs.Int("ingot_bf16", 0) != 0;
            *out = std::move(op);
            return INGOT_OK;
        });
        // ops/quant.go:941-949
        Register("", "MatMulInteger", 10, [](const NodeInfo& n, std::unique_ptr<Op>* out) {
            auto op = std::make_unique<MatMulIntegerOp>();
            op->n = n;
            op->s = t_build_session;
            *out = std::move(op);
            return INGOT_OK;
        });
        Register("", "QLinearMatMul", 10, [](const NodeInfo& n, std::unique_ptr<Op>* out) {
            auto op = std::make_unique<MatMulIntegerOp>();
            op->n = n;
            op->requant = true;
            op->s = t_build_session;
            *out = std::move(op);
            return INGOT_OK;
        });
        Register("", "QLinearConv", 10, [](const NodeInfo& n, std::unique_ptr<Op>* out) {
            auto op = std::make_unique<QLinearConvOp>();
            op->n = n;
            op->s = t_build_session;
            int rc = op->build();
            if (rc) return rc;
            *out = std::move(op);
            return INGOT_OK;
        });
        Register("", "DequantizeLinear", 10, [](const NodeInfo& n, std::unique_ptr<Op>* out) {
            auto op = std::make_unique<DequantizeLinearOp>();
            op->n = n;
            op->axis = n.attrs.Int("axis", 1);
            op->s = t_build_session;
            *out = std::move(op);
            return INGOT_OK;
        });
        // ops/elementwise.go:492-545
        auto unary = [](int act, float a, float b) {
            return [act, a, b](const NodeInfo& n, std::unique_ptr<Op>* out) {
                auto op = std::make_unique<UnaryOp>();
                op->n = n;
                op->act = act;
                op->a = a;
                op->b = b;
                op->s = t_build_session;
                *out = std::move(op);
                return INGOT_OK;
            };
        };
        Register("", "Relu", 6, unary(INGOT_ACT_RELU, 0, 0));
        Register("", "Sigmoid", 6, unary(INGOT_ACT_SIGMOID, 0, 0));
        Register("", "HardSwish", 14, unary(INGOT_ACT_HARDSWISH, 0, 0));
        Register("ingot", "HardSwish", 1, unary(INGOT_ACT_HARDSWISH, 0, 0));
        Register("ingot", "SiLU", 1, unary(INGOT_ACT_SILU, 0, 0));
        Register("ingot", "Gelu", 1, unary(INGOT_ACT_GELU_ERF, 0, 0));
        Register("", "Gelu", 20, [](const NodeInfo& n, std::unique_ptr<Op>* out) {
            auto op = std::make_unique<UnaryOp>();
            op->n = n;
            op->act = n.attrs.String("approximate", "none") == "tanh" ? INGOT_ACT_GELU_TANH : INGOT_ACT_GELU_ERF;
            op->s = t_build_session;
            *out = std::move(op);
            return INGOT_OK;
        });
        Register("", "LeakyRelu", 6, [](const NodeInfo& n, std::unique_ptr<Op>* out) {
            auto op = std::make_unique<UnaryOp>();
            op->n = n;
            op->act = INGOT_ACT_LEAKYRELU;
            op->a = n.attrs.Float("alpha", 0.01f);
            op->s = t_build_session;
            *out = std::move(op);
            return INGOT_OK;
        });
        Register("", "HardSigmoid", 6, [](const NodeInfo& n, std::unique_ptr<Op>* out) {
            auto op = std::make_unique<UnaryOp>();
            op->n = n;
            op->act = INGOT_ACT_HARDSIGMOID;
            op->a = n.attrs.Float("alpha", 0.2f);
            op->b = n.attrs.Float("beta", 0.5f);
            op->s = t_build_session;
            *out = std::move(op);
            return INGOT_OK;
        });
    });
}

}  // namespace ops
}  // namespace ingot

struct ingot_rocm_op {
    ingot_rocm_session* s;
    std::unique_ptr<ingot::ops::Op> op;
};

namespace ingot {
int op_plan(ingot_rocm_op* op, int fused_act, bool half, bool out_bf16) {
    if (!op) return fail(INGOT_EINVAL, "nil op");
    return op->op->plan(fused_act, half, out_bf16);
}
}  // namespace ingot

using namespace ingot;

extern "C" {

int ingot_rocm_op_create(ingot_rocm_session* s, const char* domain, const char* op_type, int opset, const char* attrs,
                         ingot_rocm_op** out) {
    int rc = session_enter(s);
    if (rc) return rc;
    if (!op_type || !out) return fail(INGOT_EINVAL, "nil argument");
    *out = nullptr;
    ops::register_all();
    ops::NodeInfo n;
    n.name = op_type;
    n.op_type = op_type;
    n.domain = domain ? domain : "";
    n.version = opset;
    rc = ops::parse_attrs(attrs, &n.attrs);
    if (rc) return rc;
    ops::Builder b;
    rc = ops::Lookup(n.domain, n.op_type, opset, &b);
    if (rc) return rc;
    std::unique_ptr<ops::Op> op;
    ops::t_build_session = s;
    rc = b(n, &op);
    ops::t_build_session = nullptr;
    if (rc) return rc;
    auto* h = new ingot_rocm_op();
    h->s = s;
    h->op = std::move(op);
    *out = h;
    return INGOT_OK;
}

int ingot_rocm_op_run(ingot_rocm_op* op, int n_in, const ingot_rocm_tensor* in, int max_out, ingot_rocm_tensor* out,
                      int* n_out) {
    if (!op) return fail(INGOT_EINVAL, "nil op");
    int rc = session_enter(op->s);
    if (rc) return rc;
    if (n_in < 0 || (n_in > 0 && !in) || !n_out || (max_out > 0 && !out)) return fail(INGOT_EINVAL, "bad arguments");
    std::vector<ops::T> ts(n_in);
    for (int i = 0; i < n_in; ++i) {
        if (in[i].rank < 0 || in[i].rank > 8) return fail(INGOT_EINVAL, "input %d: rank %d", i, in[i].rank);
        ts[i].dtype = in[i].dtype;
        ts[i].shape.assign(in[i].dims, in[i].dims + in[i].rank);
        ts[i].data = in[i].data;
        for (auto d : ts[i].shape)
            if (d < 0) return fail(INGOT_EINVAL, "input %d: negative dimension", i);
    }
    std::vector<ingot_rocm_tensor> outs;
    ops::Ctx ctx{op->s, &outs};
    rc = op->op->run(ctx, ts);
    if (rc) {
        for (auto& o : outs) pool_put(op->s, o.data);
        return rc;
    }
    if ((int)outs.size() > max_out) {
        for (auto& o : outs) pool_put(op->s, o.data);
        return fail(INGOT_EINVAL, "op produced %zu outputs, room for %d", outs.size(), max_out);
    }
    for (size_t i = 0; i < outs.size(); ++i) out[i] = outs[i];
    *n_out = (int)outs.size();
    return INGOT_OK;
}

int ingot_rocm_op_set_const(ingot_rocm_op* op, int input, int is_const) {
    if (!op) return fail(INGOT_EINVAL, "nil op");
    if (input < 0 || input >= 64) return fail(INGOT_EINVAL, "input index %d out of range", input);
    auto& c = op->op->const_in;
    if ((int)c.size() <= input) c.resize(input + 1, 0);
    c[input] = is_const ? 1 : 0;
    return INGOT_OK;
}

int ingot_rocm_op_free(ingot_rocm_op* op) {
    if (!op) return INGOT_OK;
    (void)session_enter(op->s);
    delete op;
    return INGOT_OK;
}

int ingot_rocm_tensor_release(ingot_rocm_session* s, ingot_rocm_tensor* t) {
    int rc = session_enter(s);
    if (rc) return rc;
    if (!t || !t->data) return INGOT_OK;
    pool_put(s, t->data);
    t->data = nullptr;
    return INGOT_OK;
}

}  // extern "C"
