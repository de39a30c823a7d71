// Graph rewrites applied to a fused node's subgraph at Compile, before its
// constants are copied to HBM. Each one merges nodes whose launches a decode
// step would otherwise pay for separately; the executor keeps an unfused path
// for every merged node, used when the fused kernel does not apply (prefill
// rows, fp32, K beyond the decode kernel's staging).
//
//  1. Sigmoid(g) -> Mul(g, .) -> Mul(., u)           => SwiGLU(g, u)
//  2. MatMulNBits q/k/v on one input, feeding one GroupQueryAttention
//                                                   => one MatMulNBits with the
//     rows concatenated, feeding GroupQueryAttention's packed-QKV form
//  3. MatMulNBits gate/up on one input, feeding SwiGLU
//                                                   => MatMulNBitsSwiGLU with
//     gate and up rows interleaved (row 2i gate i, row 2i+1 up i)
//  4. (Skip)SimplifiedLayerNormalization whose output feeds one MatMulNBits(-SwiGLU)
//                                                   => the norm runs as that
//     node's prologue (attributes __norm / __norm_eps, skip and gamma as inputs
//     6 and 7, the residual sum as output 1)
//  5. GroupQueryAttention whose output feeds one plain MatMulNBits and nothing
//     else                                          => at one-token decode steps
//     the attention leaves its split partials and the MatMulNBits merges them in
//     its prologue (attributes __partials / __merge); other steps run unfused
#include <algorithm>
#include <map>
#include <set>

#include "ep_internal.h"

namespace ortmi_ep {

namespace {

std::map<std::string, int> count_uses(const GraphIR& g, const std::vector<std::string>& outputs) {
    std::map<std::string, int> uses;
    for (const auto& n : g.nodes)
        for (const auto& in : n.inputs)
            if (!in.empty()) uses[in]++;
    for (const auto& o : outputs) uses[o] += 1000;  // fused-node outputs stay materialised
    return uses;
}

int producer_of(const GraphIR& g, const std::vector<bool>& dead, const std::string& v) {
    if (v.empty()) return -1;
    for (size_t i = 0; i < g.nodes.size(); ++i) {
        if (dead[i]) continue;
        for (const auto& o : g.nodes[i].outputs)
            if (o == v) return (int)i;
    }
    return -1;
}

void drop_dead(GraphIR& g, const std::vector<bool>& dead) {
    std::vector<NodeDesc> kept;
    for (size_t i = 0; i < g.nodes.size(); ++i)
        if (!dead[i]) kept.push_back(std::move(g.nodes[i]));
    g.nodes = std::move(kept);
}

const ValueDesc* constant(const GraphIR& g, const std::string& name) {
    auto it = g.values.find(name);
    if (it == g.values.end() || !it->second.is_initializer) return nullptr;
    return &it->second;
}

// A 4-bit MatMulNBits whose weights are constants, with no g_idx/bias input.
bool plain_mnb(const NodeDesc& n, const GraphIR& g) {
    if (n.op != "MatMulNBits" || n.attr_int("bits", 4) != 4) return false;
    for (size_t i = 4; i < n.inputs.size(); ++i)
        if (n.has_input(i)) return false;
    if (!constant(g, n.inputs[1]) || !constant(g, n.inputs[2])) return false;
    if (n.has_input(3) && !constant(g, n.inputs[3])) return false;
    return n.outputs.size() == 1 && !n.outputs[0].empty();
}

// Same activation, K, block size, zero-point presence and scale dtype.
bool mnb_compatible(const NodeDesc& a, const NodeDesc& b, const GraphIR& g) {
    return a.inputs[0] == b.inputs[0] && a.attr_int("K", 0) == b.attr_int("K", 0) &&
           a.attr_int("block_size", 32) == b.attr_int("block_size", 32) &&
           a.has_input(3) == b.has_input(3) &&
           constant(g, a.inputs[2])->dtype == constant(g, b.inputs[2])->dtype;
}

Attr int_attr(int64_t v) {
    Attr a;
    a.type = ORT_OP_ATTR_INT;
    a.i = v;
    return a;
}
Attr float_attr(float v) {
    Attr a;
    a.type = ORT_OP_ATTR_FLOAT;
    a.f = v;
    return a;
}

ValueDesc make_constant(const std::string& name, int dtype, std::vector<int64_t> dims,
                        std::vector<uint8_t> data) {
    ValueDesc v;
    v.name = name;
    v.dtype = dtype;
    v.dims = std::move(dims);
    v.has_shape = true;
    v.is_initializer = true;
    v.data = std::move(data);
    return v;
}

// Weights of one merged MatMulNBits. Each source's B / scales / zero points are
// split into per-row records of row_bytes each; `order` lists (source, row).
struct MergedWeights {
    std::vector<uint8_t> B, S, Z;
};
MergedWeights merge_rows(const GraphIR& g, const std::vector<const NodeDesc*>& src,
                         const std::vector<std::pair<int, int64_t>>& order) {
    const NodeDesc& n0 = *src[0];
    const int64_t K = n0.attr_int("K", 0), bs = n0.attr_int("block_size", 32);
    const int64_t nb = (K + bs - 1) / bs;
    const size_t brow = (size_t)nb * (size_t)bs / 2;
    const size_t srow = (size_t)nb * dtype_size(constant(g, n0.inputs[2])->dtype);
    const size_t zrow = (size_t)(nb + 1) / 2;
    const bool zp = n0.has_input(3);
    MergedWeights m;
    m.B.reserve(order.size() * brow);
    m.S.reserve(order.size() * srow);
    for (auto [s, r] : order) {
        const NodeDesc& n = *src[s];
        const auto& B = constant(g, n.inputs[1])->data;
        const auto& S = constant(g, n.inputs[2])->data;
        m.B.insert(m.B.end(), B.begin() + r * brow, B.begin() + (r + 1) * brow);
        m.S.insert(m.S.end(), S.begin() + r * srow, S.begin() + (r + 1) * srow);
        if (zp) {
            const auto& Z = constant(g, n.inputs[3])->data;
            m.Z.insert(m.Z.end(), Z.begin() + r * zrow, Z.begin() + (r + 1) * zrow);
        }
    }
    return m;
}

// True when every weight byte a merge would read is present (sizes match N, K, bs).
bool weights_complete(const NodeDesc& n, const GraphIR& g) {
    const int64_t K = n.attr_int("K", 0), N = n.attr_int("N", 0), bs = n.attr_int("block_size", 32);
    if (K <= 0 || N <= 0) return false;
    const int64_t nb = (K + bs - 1) / bs;
    const auto* B = constant(g, n.inputs[1]);
    const auto* S = constant(g, n.inputs[2]);
    if (B->data.size() != (size_t)(N * nb * bs / 2)) return false;
    if (S->data.size() != (size_t)(N * nb) * dtype_size(S->dtype)) return false;
    if (n.has_input(3) && constant(g, n.inputs[3])->data.size() != (size_t)(N * ((nb + 1) / 2)))
        return false;
    return true;
}

// Adds the merged constants and points `n` (a copy of a source node) at them.
void install_weights(GraphIR& g, NodeDesc& n, const std::string& base, MergedWeights&& m,
                     int64_t N) {
    const int64_t K = n.attr_int("K", 0), bs = n.attr_int("block_size", 32);
    const int64_t nb = (K + bs - 1) / bs;
    const int sdt = constant(g, n.inputs[2])->dtype;
    g.values[base + ".B"] = make_constant(base + ".B", ONNX_TENSOR_ELEMENT_DATA_TYPE_UINT8,
                                          {N, nb, bs / 2}, std::move(m.B));
    g.values[base + ".scales"] = make_constant(base + ".scales", sdt, {N * nb}, std::move(m.S));
    n.inputs[1] = base + ".B";
    n.inputs[2] = base + ".scales";
    if (n.has_input(3)) {
        g.values[base + ".zp"] = make_constant(base + ".zp", ONNX_TENSOR_ELEMENT_DATA_TYPE_UINT8,
                                               {N * ((nb + 1) / 2)}, std::move(m.Z));
        n.inputs[3] = base + ".zp";
    }
    n.attrs["N"] = int_attr(N);
}

// Removes constants no node reads any more.
void drop_unused_constants(GraphIR& g) {
    std::set<std::string> used;
    for (const auto& n : g.nodes)
        for (const auto& in : n.inputs)
            if (!in.empty()) used.insert(in);
    for (auto it = g.values.begin(); it != g.values.end();) {
        if (it->second.is_initializer && !used.count(it->first)) it = g.values.erase(it);
        else ++it;
    }
}

void fuse_swiglu(GraphIR& g, const std::vector<std::string>& outputs) {
    auto uses = count_uses(g, outputs);
    auto other = [](const NodeDesc& m, const std::string& x) -> std::string {
        if (m.inputs.size() != 2) return "";
        if (m.inputs[0] == x) return m.inputs[1];
        if (m.inputs[1] == x) return m.inputs[0];
        return "";
    };
    std::vector<bool> dead(g.nodes.size(), false);
    for (size_t i = 0; i < g.nodes.size(); ++i) {
        const NodeDesc& sg = g.nodes[i];
        if (sg.op != "Sigmoid" || sg.domain != "" || sg.outputs.empty()) continue;
        const std::string x = sg.inputs[0], s = sg.outputs[0];
        if (uses[s] != 1) continue;
        for (size_t j = 0; j < g.nodes.size(); ++j) {
            NodeDesc& m1 = g.nodes[j];
            if (dead[j] || m1.op != "Mul" || other(m1, s) != x || m1.outputs.empty()) continue;
            const std::string t = m1.outputs[0];
            if (uses[t] != 1) break;
            for (size_t k = 0; k < g.nodes.size(); ++k) {
                NodeDesc& m2 = g.nodes[k];
                if (dead[k] || m2.op != "Mul") continue;
                const std::string u = other(m2, t);
                if (u.empty() || u == t) continue;
                const auto vx = g.values.find(x), vu = g.values.find(u);
                if (vx == g.values.end() || vu == g.values.end() ||
                    vx->second.dims != vu->second.dims)
                    break;
                m2.op = "SwiGLU";
                m2.domain = "";
                m2.inputs = {x, u};
                dead[i] = dead[j] = true;
                break;
            }
            break;
        }
    }
    drop_dead(g, dead);
}

void fuse_qkv(GraphIR& g, const std::vector<std::string>& outputs) {
    auto uses = count_uses(g, outputs);
    std::vector<bool> dead(g.nodes.size(), false);
    for (size_t gi = 0; gi < g.nodes.size(); ++gi) {
        NodeDesc& attn = g.nodes[gi];
        if (attn.op != "GroupQueryAttention" || !attn.has_input(1) || !attn.has_input(2)) continue;
        int p[3];
        bool ok = true;
        for (int i = 0; i < 3 && ok; ++i) {
            p[i] = producer_of(g, dead, attn.inputs[i]);
            ok = p[i] >= 0 && plain_mnb(g.nodes[p[i]], g) && uses[attn.inputs[i]] == 1 &&
                 weights_complete(g.nodes[p[i]], g);
        }
        if (!ok || p[0] == p[1] || p[1] == p[2] || p[0] == p[2]) continue;
        const NodeDesc &q = g.nodes[p[0]], &k = g.nodes[p[1]], &v = g.nodes[p[2]];
        if (!mnb_compatible(q, k, g) || !mnb_compatible(q, v, g)) continue;
        std::vector<const NodeDesc*> src = {&q, &k, &v};
        std::vector<std::pair<int, int64_t>> order;
        int64_t N = 0;
        for (int s = 0; s < 3; ++s) {
            const int64_t ns = src[s]->attr_int("N", 0);
            for (int64_t r = 0; r < ns; ++r) order.emplace_back(s, r);
            N += ns;
        }
        NodeDesc merged = q;
        merged.name = q.name + "/qkv";
        const std::string out = attn.name + "/qkv_packed";
        install_weights(g, merged, merged.name, merge_rows(g, src, order), N);
        merged.outputs = {out};
        ValueDesc ov = g.values.at(attn.inputs[0]);
        ov.name = out;
        if (!ov.dims.empty() && ov.dims.back() >= 0) ov.dims.back() = N;
        g.values[out] = ov;
        attn.inputs[0] = out;
        attn.inputs[1].clear();
        attn.inputs[2].clear();
        g.nodes[p[0]] = std::move(merged);
        dead[p[1]] = dead[p[2]] = true;
    }
    drop_dead(g, dead);
}

void fuse_gate_up(GraphIR& g, const std::vector<std::string>& outputs) {
    auto uses = count_uses(g, outputs);
    std::vector<bool> dead(g.nodes.size(), false);
    for (size_t wi = 0; wi < g.nodes.size(); ++wi) {
        NodeDesc& w = g.nodes[wi];
        if (w.op != "SwiGLU" || w.inputs.size() != 2) continue;
        const int pg = producer_of(g, dead, w.inputs[0]), pu = producer_of(g, dead, w.inputs[1]);
        if (pg < 0 || pu < 0 || pg == pu) continue;
        const NodeDesc &gate = g.nodes[pg], &up = g.nodes[pu];
        if (!plain_mnb(gate, g) || !plain_mnb(up, g) || !mnb_compatible(gate, up, g)) continue;
        if (uses[w.inputs[0]] != 1 || uses[w.inputs[1]] != 1) continue;
        if (!weights_complete(gate, g) || !weights_complete(up, g)) continue;
        const int64_t N = gate.attr_int("N", 0);
        if (up.attr_int("N", 0) != N) continue;
        std::vector<const NodeDesc*> src = {&gate, &up};
        std::vector<std::pair<int, int64_t>> order;
        for (int64_t r = 0; r < N; ++r) {
            order.emplace_back(0, r);
            order.emplace_back(1, r);
        }
        NodeDesc merged = gate;
        merged.op = "MatMulNBitsSwiGLU";
        merged.domain = "";
        merged.name = gate.name + "/gate_up";
        install_weights(g, merged, merged.name, merge_rows(g, src, order), 2 * N);
        merged.outputs = {w.outputs[0]};
        g.nodes[pg] = std::move(merged);
        dead[pu] = dead[wi] = true;
    }
    drop_dead(g, dead);
}

void fuse_norm_prologue(GraphIR& g, const std::vector<std::string>& outputs) {
    auto uses = count_uses(g, outputs);
    std::vector<bool> dead(g.nodes.size(), false);
    for (size_t ni = 0; ni < g.nodes.size(); ++ni) {
        const NodeDesc& nn = g.nodes[ni];
        const bool skip = nn.op == "SkipSimplifiedLayerNormalization";
        if (!(skip || nn.op == "SimplifiedLayerNormalization") || nn.outputs.empty()) continue;
        if (nn.attr_int("axis", -1) != -1) continue;
        if (skip && nn.has_input(3)) continue;  // bias
        const std::string y = nn.outputs[0];
        if (y.empty() || uses[y] != 1) continue;
        int ci = -1;
        for (size_t j = 0; j < g.nodes.size(); ++j)
            if (!dead[j] && !g.nodes[j].inputs.empty() && g.nodes[j].inputs[0] == y) ci = (int)j;
        if (ci < 0) continue;
        NodeDesc& c = g.nodes[ci];
        if (c.op != "MatMulNBits" && c.op != "MatMulNBitsSwiGLU") continue;
        if (!plain_mnb(c, g) && c.op == "MatMulNBits") continue;
        if (c.attr_int("__norm", 0)) continue;
        c.inputs[0] = nn.inputs[0];
        c.inputs.resize(8);
        c.inputs[6] = skip ? nn.inputs[1] : std::string();
        c.inputs[7] = skip ? nn.inputs[2] : nn.inputs[1];
        c.attrs["__norm"] = int_attr(1);
        c.attrs["__norm_eps"] = float_attr(nn.attr_float("epsilon", skip ? 1e-6f : 1e-5f));
        c.outputs.resize(2);
        c.outputs[1] = (skip && nn.outputs.size() >= 4) ? nn.outputs[3] : std::string();
        dead[ni] = true;
    }
    drop_dead(g, dead);
}

void mark_attention_merge(GraphIR& g, const std::vector<std::string>& outputs) {
    auto uses = count_uses(g, outputs);
    for (auto& n : g.nodes) {
        if (n.op != "GroupQueryAttention" || n.outputs.empty() || n.outputs[0].empty()) continue;
        if (n.attr_int("sliding_window_cache", 0)) continue;  // its output is always whole
        const std::string& y = n.outputs[0];
        if (uses[y] != 1) continue;
        const int64_t H = n.attr_int("num_heads", 0);
        for (auto& c : g.nodes) {
            if (c.op != "MatMulNBits" || c.inputs.empty() || c.inputs[0] != y) continue;
            if (!plain_mnb(c, g) || c.attr_int("__norm", 0)) continue;
            const int64_t K = c.attr_int("K", 0), bs = c.attr_int("block_size", 32);
            const int sdt = constant(g, c.inputs[2])->dtype;
            const bool half_scales = sdt == ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT16 ||
                                     sdt == ONNX_TENSOR_ELEMENT_DATA_TYPE_BFLOAT16;
            const int64_t hd = H > 0 && K % H == 0 ? K / H : 0;
            // The merge GEMV's form: 4-bit, block 32-128, K within its staging,
            // fp16/bf16, head size 64 or 128.
            if (!half_scales || (bs != 32 && bs != 64 && bs != 128) || K > 10240 ||
                (hd != 64 && hd != 128))
                continue;
            n.attrs["__partials"] = int_attr(1);
            c.attrs["__merge"] = int_attr(1);
        }
    }
}

// Stable topological order (a merged node may now produce a value that an
// earlier node in the old order reads).
void topo_sort(GraphIR& g) {
    const size_t N = g.nodes.size();
    std::map<std::string, size_t> producer;
    for (size_t i = 0; i < N; ++i)
        for (const auto& o : g.nodes[i].outputs)
            if (!o.empty()) producer[o] = i;
    std::vector<std::vector<size_t>> succ(N);
    std::vector<int> indeg(N, 0);
    for (size_t i = 0; i < N; ++i) {
        std::set<size_t> seen;
        for (const auto& in : g.nodes[i].inputs) {
            auto it = in.empty() ? producer.end() : producer.find(in);
            if (it != producer.end() && it->second != i && seen.insert(it->second).second) {
                succ[it->second].push_back(i);
                indeg[i]++;
            }
        }
    }
    std::set<size_t> ready;
    for (size_t i = 0; i < N; ++i)
        if (!indeg[i]) ready.insert(i);
    std::vector<size_t> order;
    while (!ready.empty()) {
        const size_t v = *ready.begin();
        ready.erase(ready.begin());
        order.push_back(v);
        for (size_t s : succ[v])
            if (--indeg[s] == 0) ready.insert(s);
    }
    if (order.size() != N) fail("fused subgraph has a cycle after rewriting", ORT_INVALID_GRAPH);
    std::vector<NodeDesc> sorted;
    sorted.reserve(N);
    for (size_t i : order) sorted.push_back(std::move(g.nodes[i]));
    g.nodes = std::move(sorted);
}

}  // namespace

void fuse_subgraph(GraphIR& g, const std::vector<std::string>& outputs, bool decode_fusions) {
    fuse_swiglu(g, outputs);
    if (decode_fusions) {
        fuse_qkv(g, outputs);
        fuse_gate_up(g, outputs);
        fuse_norm_prologue(g, outputs);
        mark_attention_merge(g, outputs);
        drop_unused_constants(g);
    }
    topo_sort(g);
}

}  // namespace ortmi_ep
