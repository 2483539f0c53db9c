// Graph session: an ONNX node list compiled and run on the operator layer,
// planned the way the reference's GPU session plans this path.
//
//  - fuseMatMulBias (graph/fuse_matmul_bias.go:12-63): MatMul(x, W) →
//    Add(·, bias), W a constant f32 2-D weight and bias a constant f32 [N]
//    broadcast over rows, becomes a 3-input MatMul (bias in the GEMM store).
//  - planHalf (graph/gpuhalf_darwin_arm64.go:29-112): a Gemm / MatMul against
//    a constant weight whose only consumer (slot 0) is Relu, Sigmoid, SiLU or
//    Gelu (erf / tanh) applies it in its store, and the activation node
//    passes its input through; under GPUBF16 (graph/device.go:20-30) every
//    product against a constant weight runs in bf16, and a product whose
//    value is read only by such products (as their A) stores it in bf16.
//
// Steps run in node order on the session stream; intermediate values live
// in the session pool and go back to it after their last reader is queued
// (stream order makes the reuse safe). Graph outputs are always f32 pool
// tensors, released by the caller with ingot_rocm_tensor_release — the
// reference's Session.Release (graph/session.go).
//
// Text form (one statement per line, '#' starts a comment):
//   input  <name> <dtype> [<d0,d1,...> | ?]
//   const  <name> <dtype> <d0,d1,...>          (device data: ingot_rocm_graph_bind)
//   node   [<domain>.]<op>[@<opset>] <in,in,...|_> -> <out,...> [<attrs>]
//   output <name>
// dtype: f32 bf16 f16 i8 u8 i16 i32 i64 bool; an absent optional input is
// '_'; attrs as for ingot_rocm_op_create ("i:transB=1;f:alpha=0.5").

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "runtime.hpp"

namespace ingot {
namespace graph {

struct Value {
    std::string name;
    int dtype = 0;
    std::vector<int64_t> shape;
    bool has_shape = false;
    bool is_const = false, is_input = false, is_output = false;
    ingot_rocm_tensor bound;
    bool is_bound = false;
    int producer = -1;
    std::vector<std::pair<int, int>> users;  // (node, slot) of live nodes
};

struct Node {
    std::string domain, op, attrs;
    int opset = 0;
    std::vector<int> in;  // -1: absent optional input
    std::vector<int> out;
    bool dead = false;
    int fused_act = INGOT_ACT_NONE;
    bool half = false, half_out = false, pass = false;
    ingot_rocm_op* impl = nullptr;
};

int dtype_code(const std::string& s) {
    static const std::map<std::string, int> m = {
        {"f32", INGOT_DT_F32}, {"f16", INGOT_DT_F16}, {"bf16", INGOT_DT_BF16}, {"i8", INGOT_DT_I8},
        {"u8", INGOT_DT_U8},   {"i16", INGOT_DT_I16}, {"i32", INGOT_DT_I32},   {"i64", INGOT_DT_I64},
        {"bool", INGOT_DT_BOOL}};
    auto it = m.find(s);
    return it == m.end() ? 0 : it->second;
}

std::vector<std::string> split(const std::string& s, char sep) {
    std::vector<std::string> r;
    size_t p = 0;
    while (true) {
        size_t q = s.find(sep, p);
        r.push_back(s.substr(p, q == std::string::npos ? std::string::npos : q - p));
        if (q == std::string::npos) break;
        p = q + 1;
    }
    return r;
}

}  // namespace graph
}  // namespace ingot

struct ingot_rocm_graph {
    ingot_rocm_session* s = nullptr;
    std::vector<ingot::graph::Value> vals;
    std::map<std::string, int> ids;
    std::vector<ingot::graph::Node> nodes;
    std::vector<int> outputs;
    std::map<std::string, int> stats;
    int flags = 0;
    bool compiled = false;
};

namespace ingot {
namespace graph {

int value_id(ingot_rocm_graph* g, const std::string& name) {
    auto it = g->ids.find(name);
    if (it != g->ids.end()) return it->second;
    Value v;
    v.name = name;
    g->vals.push_back(v);
    const int id = (int)g->vals.size() - 1;
    g->ids[name] = id;
    return id;
}

int parse_dims(const std::string& t, Value* v, int line) {
    if (t == "?") return INGOT_OK;
    v->has_shape = true;
    v->shape.clear();
    if (t == "scalar") return INGOT_OK;
    for (auto& d : split(t, ',')) {
        char* ep = nullptr;
        const long long x = strtoll(d.c_str(), &ep, 10);
        if (d.empty() || *ep || x < 0) return fail(INGOT_EINVAL, "graph line %d: bad dimension list \"%s\"", line, t.c_str());
        v->shape.push_back(x);
    }
    return INGOT_OK;
}

int parse(ingot_rocm_graph* g, const char* text) {
    std::istringstream in(text ? text : "");
    std::string line;
    int ln = 0;
    while (std::getline(in, line)) {
        ++ln;
        const size_t hash = line.find('#');
        if (hash != std::string::npos) line.resize(hash);
        std::istringstream ls(line);
        std::vector<std::string> tok;
        for (std::string t; ls >> t;) tok.push_back(t);
        if (tok.empty()) continue;
        const std::string& kw = tok[0];
        if (kw == "input" || kw == "const") {
            if (tok.size() < 3 || tok.size() > 4 || (kw == "const" && tok.size() != 4))
                return fail(INGOT_EINVAL, "graph line %d: %s <name> <dtype> %s", ln, kw.c_str(),
                            kw == "const" ? "<dims>" : "[<dims>]");
            const int id = value_id(g, tok[1]);
            Value& v = g->vals[id];
            if (v.is_input || v.is_const || v.producer >= 0)
                return fail(INGOT_EINVAL, "graph line %d: value \"%s\" defined twice", ln, tok[1].c_str());
            v.dtype = dtype_code(tok[2]);
            if (!v.dtype) return fail(INGOT_EINVAL, "graph line %d: unknown dtype \"%s\"", ln, tok[2].c_str());
            (kw == "input" ? v.is_input : v.is_const) = true;
            if (tok.size() == 4) {
                int rc = parse_dims(tok[3], &v, ln);
                if (rc) return rc;
            }
        } else if (kw == "output") {
            if (tok.size() != 2) return fail(INGOT_EINVAL, "graph line %d: output <name>", ln);
            auto it = g->ids.find(tok[1]);
            if (it == g->ids.end() || g->vals[it->second].producer < 0)
                return fail(INGOT_EINVAL, "graph line %d: output \"%s\" is not produced by a node", ln, tok[1].c_str());
            g->vals[it->second].is_output = true;
            g->outputs.push_back(it->second);
        } else if (kw == "node") {
            if (tok.size() < 5 || tok.size() > 6 || tok[3] != "->")
                return fail(INGOT_EINVAL, "graph line %d: node <op> <inputs> -> <outputs> [attrs]", ln);
            Node n;
            std::string spec = tok[1];
            const size_t at = spec.find('@');
            if (at != std::string::npos) {
                n.opset = atoi(spec.c_str() + at + 1);
                spec.resize(at);
            }
            const size_t dot = spec.rfind('.');
            if (dot != std::string::npos) {
                n.domain = spec.substr(0, dot);
                n.op = spec.substr(dot + 1);
            } else {
                n.op = spec;
            }
            if (!n.opset) n.opset = n.domain.empty() ? 13 : 1;
            const int self = (int)g->nodes.size();
            for (auto& name : split(tok[2], ',')) {
                if (name == "_") {
                    n.in.push_back(-1);
                    continue;
                }
                auto it = g->ids.find(name);
                if (it == g->ids.end() ||
                    !(g->vals[it->second].is_input || g->vals[it->second].is_const || g->vals[it->second].producer >= 0))
                    return fail(INGOT_EINVAL, "graph line %d: input \"%s\" is not defined before its use", ln,
                                name.c_str());
                n.in.push_back(it->second);
            }
            for (auto& name : split(tok[4], ',')) {
                const int id = value_id(g, name);
                Value& v = g->vals[id];
                if (v.is_input || v.is_const || v.producer >= 0)
                    return fail(INGOT_EINVAL, "graph line %d: value \"%s\" defined twice", ln, name.c_str());
                v.producer = self;
                n.out.push_back(id);
            }
            if (tok.size() == 6) n.attrs = tok[5];
            g->nodes.push_back(n);
        } else {
            return fail(INGOT_EINVAL, "graph line %d: unknown statement \"%s\"", ln, kw.c_str());
        }
    }
    if (g->outputs.empty()) return fail(INGOT_EINVAL, "graph: no outputs");
    return INGOT_OK;
}

void link_users(ingot_rocm_graph* g) {
    for (auto& v : g->vals) v.users.clear();
    for (size_t i = 0; i < g->nodes.size(); ++i) {
        const Node& n = g->nodes[i];
        if (n.dead) continue;
        for (size_t k = 0; k < n.in.size(); ++k)
            if (n.in[k] >= 0) g->vals[n.in[k]].users.push_back({(int)i, (int)k});
    }
}

// soleConsumer (graph/optimize.go:123-128)
int sole_consumer(const ingot_rocm_graph* g, int id) {
    const Value& v = g->vals[id];
    if (v.users.size() != 1 || v.is_output) return -1;
    return v.users[0].first;
}

// constWeight (graph/gpuhalf_darwin_arm64.go:45-51)
bool const_weight(const ingot_rocm_graph* g, const Node& n) {
    if (n.in.size() < 2 || n.in[1] < 0) return false;
    const Value& w = g->vals[n.in[1]];
    return w.is_const && w.dtype == INGOT_DT_F32 && w.has_shape && w.shape.size() == 2;
}

bool is_product(const Node& n) { return n.domain.empty() && (n.op == "Gemm" || n.op == "MatMul"); }

bool matmul_gelu(const Node& n) { return n.op == "MatMul" && n.attrs.find("s:ingot_act=gelu") != std::string::npos; }

// unaryAct (graph/gpuhalf_darwin_arm64.go:118-123) over the ONNX nodes that
// map to those GPU unary ops.
int unary_act(const Node& n) {
    if (n.domain.empty() && n.op == "Relu") return INGOT_ACT_RELU;
    if (n.domain.empty() && n.op == "Sigmoid") return INGOT_ACT_SIGMOID;
    if (n.domain == "ingot" && n.op == "SiLU") return INGOT_ACT_SILU;
    if (n.domain == "ingot" && n.op == "Gelu") return INGOT_ACT_GELU_ERF;
    if (n.domain.empty() && n.op == "Gelu")
        return n.attrs.find("s:approximate=tanh") != std::string::npos ? INGOT_ACT_GELU_TANH : INGOT_ACT_GELU_ERF;
    return INGOT_ACT_NONE;
}

// fuseMatMulBias (graph/fuse_matmul_bias.go:12-63)
void fuse_matmul_bias(ingot_rocm_graph* g) {
    link_users(g);
    for (size_t i = 0; i < g->nodes.size(); ++i) {
        Node& mm = g->nodes[i];
        if (mm.dead || mm.op != "MatMul" || !mm.domain.empty() || mm.in.size() != 2) continue;
        if (!const_weight(g, mm)) continue;
        const int64_t n = g->vals[mm.in[1]].shape[1];
        const int mid = mm.out[0];
        const int ai = sole_consumer(g, mid);
        if (ai < 0) continue;
        Node& add = g->nodes[ai];
        if (add.dead || add.op != "Add" || !add.domain.empty() || add.in.size() != 2) continue;
        int bias = -1;
        if (add.in[0] == mid && add.in[1] >= 0 && g->vals[add.in[1]].is_const) bias = add.in[1];
        else if (add.in[1] == mid && add.in[0] >= 0 && g->vals[add.in[0]].is_const) bias = add.in[0];
        if (bias < 0) continue;
        const Value& b = g->vals[bias];
        int64_t bn = 1;
        for (auto d : b.shape) bn *= d;
        if (b.dtype != INGOT_DT_F32 || !b.has_shape || bn != n || b.shape.empty() || b.shape.back() != n) continue;
        const Value& mv = g->vals[mid];
        if (mv.has_shape && b.shape.size() > mv.shape.size()) continue;
        mm.in.push_back(bias);
        mm.out = add.out;
        g->vals[add.out[0]].producer = (int)i;
        add.dead = true;
        g->stats["fuse-matmul-bias"]++;
        link_users(g);
    }
}

// planHalf (graph/gpuhalf_darwin_arm64.go:29-112): epilogue activations and,
// under GPUBF16, bf16 products and bf16-resident values.
void plan_half(ingot_rocm_graph* g, bool fuse_act, bool bf16) {
    link_users(g);
    auto out0 = [&](int i) { return g->nodes[i].out.empty() ? -1 : g->nodes[i].out[0]; };
    std::vector<int> act_user(g->nodes.size(), -1);
    if (fuse_act) {
        for (size_t i = 0; i < g->nodes.size(); ++i) {
            Node& n = g->nodes[i];
            if (n.dead || !is_product(n) || matmul_gelu(n) || !const_weight(g, n)) continue;
            const int id = out0((int)i);
            const Value& v = g->vals[id];
            if (id < 0 || v.is_output || v.users.size() != 1 || v.users[0].second != 0) continue;
            const int u = v.users[0].first;
            const int act = unary_act(g->nodes[u]);
            if (act == INGOT_ACT_NONE || out0(u) < 0) continue;
            n.fused_act = act;
            g->nodes[u].pass = true;
            act_user[i] = u;
            g->stats["fuse-act"]++;
        }
    }
    if (!bf16) return;
    // want[id]: 0 unknown, 1 every reader takes bf16, 2 not
    std::vector<int> want(g->vals.size(), 0);
    auto reads = [&](std::pair<int, int> u) {
        const Node& n = g->nodes[u.first];
        return !n.dead && !n.pass && is_product(n) && u.second == 0 && const_weight(g, n);
    };
    auto wants = [&](int id) {
        if (want[id] == 0) {
            const Value& v = g->vals[id];
            want[id] = (v.is_output || v.users.empty()) ? 2 : 1;
            for (auto& u : v.users)
                if (!reads(u)) want[id] = 2;
        }
        return want[id] == 1;
    };
    for (size_t i = 0; i < g->nodes.size(); ++i) {
        Node& n = g->nodes[i];
        if (n.dead || !is_product(n) || !const_weight(g, n)) continue;
        n.half = true;
        const int id = act_user[i] >= 0 ? out0(act_user[i]) : out0((int)i);
        if (id >= 0 && wants(id)) {
            n.half_out = true;
            g->stats["half-out"]++;
        }
    }
}

}  // namespace graph
}  // namespace ingot

using namespace ingot;
using namespace ingot::graph;

extern "C" {

int ingot_rocm_graph_create(ingot_rocm_session* s, const char* text, ingot_rocm_graph** out) {
    if (s) {
        int rc = session_enter(s);
        if (rc) return rc;
    }
    if (!out) return fail(INGOT_EINVAL, "nil out");
    *out = nullptr;
    auto* g = new ingot_rocm_graph();
    g->s = s;
    int rc = parse(g, text);
    if (rc) {
        delete g;
        return rc;
    }
    *out = g;
    return INGOT_OK;
}

int ingot_rocm_graph_bind(ingot_rocm_graph* g, const char* name, const ingot_rocm_tensor* t) {
    if (!g || !name || !t) return fail(INGOT_EINVAL, "nil argument");
    auto it = g->ids.find(name);
    if (it == g->ids.end() || !g->vals[it->second].is_const)
        return fail(INGOT_EINVAL, "graph: \"%s\" is not a declared constant", name);
    Value& v = g->vals[it->second];
    bool same = t->dtype == v.dtype && t->rank == (int)v.shape.size();
    for (int d = 0; same && d < t->rank; ++d) same = t->dims[d] == v.shape[d];
    if (!same) return fail(INGOT_EINVAL, "graph: constant \"%s\" bound with another dtype or shape", name);
    v.bound = *t;
    v.is_bound = true;
    return INGOT_OK;
}

int ingot_rocm_graph_compile(ingot_rocm_graph* g, int flags) {
    if (!g) return fail(INGOT_EINVAL, "nil graph");
    if (g->compiled) return fail(INGOT_EINVAL, "graph: already compiled");
    if (flags & ~(INGOT_GRAPH_FUSE_BIAS | INGOT_GRAPH_FUSE_ACT | INGOT_GRAPH_HALF))
        return fail(INGOT_EINVAL, "graph: unknown compile flags 0x%x", flags);
    if (g->s) {
        int rc = session_enter(g->s);
        if (rc) return rc;
        for (auto& v : g->vals)
            if (v.is_const && !v.is_bound) return fail(INGOT_EINVAL, "graph: constant \"%s\" is not bound", v.name.c_str());
    }
    g->flags = flags;
    if (flags & INGOT_GRAPH_FUSE_BIAS) fuse_matmul_bias(g);
    plan_half(g, (flags & INGOT_GRAPH_FUSE_ACT) != 0, (flags & INGOT_GRAPH_HALF) != 0);
    link_users(g);
    int steps = 0;
    for (auto& n : g->nodes) {
        if (n.dead || n.pass) continue;
        ++steps;
        if (!g->s) continue;
        std::string attrs = n.attrs;
        int rc = ingot_rocm_op_create(g->s, n.domain.c_str(), n.op.c_str(), n.opset, attrs.c_str(), &n.impl);
        if (rc) return rc;
        // bound constants keep their storage and values across runs: the op may
        // pack them once (every other operand is packed per call)
        for (size_t k = 0; k < n.in.size(); ++k)
            if (n.in[k] >= 0 && g->vals[n.in[k]].is_const && (rc = ingot_rocm_op_set_const(n.impl, (int)k, 1)))
                return rc;
        if (n.fused_act != INGOT_ACT_NONE || n.half || n.half_out) {
            rc = op_plan(n.impl, n.fused_act, n.half, n.half_out);
            if (rc) return fail(rc, "graph: %s does not take a plan", n.op.c_str());
        }
    }
    g->stats["steps"] = steps;
    g->compiled = true;
    return INGOT_OK;
}

int ingot_rocm_graph_describe(const ingot_rocm_graph* g, int what, char* buf, size_t n) {
    if (!g || !buf || !n) return fail(INGOT_EINVAL, "nil argument");
    std::string r;
    if (what == 0) {
        for (auto& kv : g->stats) r += kv.first + "=" + std::to_string(kv.second) + ";";
    } else {
        for (auto& nd : g->nodes) {
            if (nd.dead) continue;
            r += (nd.domain.empty() ? "" : nd.domain + ".") + nd.op + " in=";
            for (size_t k = 0; k < nd.in.size(); ++k)
                r += (k ? "," : "") + (nd.in[k] < 0 ? std::string("_") : g->vals[nd.in[k]].name);
            r += " out=";
            for (size_t k = 0; k < nd.out.size(); ++k) r += (k ? "," : "") + g->vals[nd.out[k]].name;
            r += " act=" + std::to_string(nd.fused_act) + " half=" + std::to_string(nd.half) +
                 " bf16_out=" + std::to_string(nd.half_out) + " pass=" + std::to_string(nd.pass) + "\n";
        }
    }
    if (r.size() + 1 > n) return fail(INGOT_EINVAL, "graph: description needs %zu bytes", r.size() + 1);
    memcpy(buf, r.c_str(), r.size() + 1);
    return INGOT_OK;
}

int ingot_rocm_graph_run(ingot_rocm_graph* g, int n_in, const char* const* names, const ingot_rocm_tensor* in,
                         int max_out, ingot_rocm_tensor* out, int* n_out) {
    if (!g || !g->compiled) return fail(INGOT_EINVAL, "graph: not compiled");
    if (!g->s) return fail(INGOT_EINVAL, "graph: planned without a session; it cannot run");
    int rc = session_enter(g->s);
    if (rc) return rc;
    if (n_in < 0 || (n_in && (!names || !in)) || !n_out || (int)g->outputs.size() > max_out || !out)
        return fail(INGOT_EINVAL, "graph: bad arguments (room for %d outputs, %zu needed)", max_out, g->outputs.size());
    const size_t nv = g->vals.size();
    std::vector<ingot_rocm_tensor> cur(nv);
    std::vector<char> have(nv, 0), owned(nv, 0);
    std::map<void*, int> refs;  // pooled storage → values holding it
    for (size_t i = 0; i < nv; ++i)
        if (g->vals[i].is_const) cur[i] = g->vals[i].bound, have[i] = 1;
    for (int i = 0; i < n_in; ++i) {
        auto it = names[i] ? g->ids.find(names[i]) : g->ids.end();
        if (it == g->ids.end() || !g->vals[it->second].is_input)
            return fail(INGOT_EINVAL, "graph: \"%s\" is not an input", names[i] ? names[i] : "(nil)");
        const Value& v = g->vals[it->second];
        if (in[i].dtype != v.dtype) return fail(INGOT_EINVAL, "graph: input \"%s\" has the wrong dtype", v.name.c_str());
        if (v.has_shape) {
            bool same = in[i].rank == (int)v.shape.size();
            for (int d = 0; same && d < in[i].rank; ++d) same = in[i].dims[d] == v.shape[d];
            if (!same) return fail(INGOT_EINVAL, "graph: input \"%s\" has the wrong shape", v.name.c_str());
        }
        cur[it->second] = in[i];
        have[it->second] = 1;
    }
    for (size_t i = 0; i < nv; ++i)
        if (g->vals[i].is_input && !have[i]) return fail(INGOT_EINVAL, "graph: input \"%s\" not fed", g->vals[i].name.c_str());
    // remaining reads per value (graph outputs keep one for the caller)
    std::vector<int> uses(nv, 0);
    for (size_t i = 0; i < nv; ++i) uses[i] = (int)g->vals[i].users.size() + (g->vals[i].is_output ? 1 : 0);
    auto drop = [&](int id) {
        if (--uses[id] > 0 || !owned[id]) return;
        void* p = cur[id].data;
        if (--refs[p] == 0) {
            (void)ingot_rocm_tensor_release(g->s, &cur[id]);
            refs.erase(p);
        }
    };
    auto release_all = [&]() {
        for (auto& kv : refs) {
            ingot_rocm_tensor t;
            memset(&t, 0, sizeof t);
            t.data = kv.first;
            (void)ingot_rocm_tensor_release(g->s, &t);
        }
        refs.clear();
    };
    for (auto& nd : g->nodes) {
        if (nd.dead) continue;
        if (nd.pass) {  // the producer applied this activation in its store
            const int src = nd.in[0], dst = nd.out[0];
            cur[dst] = cur[src];
            owned[dst] = owned[src];
            if (owned[dst]) refs[cur[dst].data]++;
            drop(src);
            continue;
        }
        std::vector<ingot_rocm_tensor> ins(nd.in.size());
        for (size_t k = 0; k < nd.in.size(); ++k) {
            if (nd.in[k] < 0) {
                memset(&ins[k], 0, sizeof ins[k]);
                continue;
            }
            ins[k] = cur[nd.in[k]];
        }
        ingot_rocm_tensor outs[8];
        int no = 0;
        rc = ingot_rocm_op_run(nd.impl, (int)ins.size(), ins.data(), 8, outs, &no);
        if (rc) {
            release_all();
            return rc;
        }
        for (int k = 0; k < no; ++k) {
            if (k < (int)nd.out.size()) {
                cur[nd.out[k]] = outs[k];
                owned[nd.out[k]] = 1;
                refs[outs[k].data]++;
            } else {
                (void)ingot_rocm_tensor_release(g->s, &outs[k]);
            }
        }
        for (int id : nd.in)
            if (id >= 0) drop(id);
    }
    for (size_t k = 0; k < g->outputs.size(); ++k) {
        const int id = g->outputs[k];
        out[k] = cur[id];
        refs.erase(cur[id].data);  // the caller's now
    }
    release_all();
    *n_out = (int)g->outputs.size();
    return INGOT_OK;
}

int ingot_rocm_graph_free(ingot_rocm_graph* g) {
    if (!g) return INGOT_OK;
    for (auto& n : g->nodes)
        if (n.impl) (void)ingot_rocm_op_free(n.impl);
    delete g;
    return INGOT_OK;
}

}  // extern "C"
