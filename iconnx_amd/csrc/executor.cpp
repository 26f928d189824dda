// Graph executor for the quantized-linear path and the encoder around it: the MI355X
// counterpart of the reference's GpuGraphExecutor shim (src/cuda/inference/mod.rs:208-659),
// its lowering (ir::lower, src/ir/lowering.rs:31-238) and per-op dispatch
// (src/cuda/executor/mod.rs:107-597).
//
//   build:   add_input / add_initializer / add_node (+ float and int-list attributes) /
//            add_output (host only)
//   plan:    requested outputs (or the graph's sinks, mod.rs:505-519) and dead-node
//            elimination; topological sort; fusion decision (host only):
//              Attention        Reshape/Transpose/MatMul/scale/Softmax/MatMul/Transpose/
//                               Reshape of a BERT self-attention -> one fused kernel
//              QuantizedLinear  MatMulInteger -> Cast -> Mul -> [Add] -> [chain] [-> GELU]
//              AddLayerNorm     LayerNormalization(Add(a, b))
//              DecomposedLayerNorm  [Add(a, b) ->] ReduceMean -> Sub -> Pow(2) -> ReduceMean
//                               -> Add(eps) -> Sqrt -> Div [-> Mul(gamma)] [-> Add(beta)]
//              MulAdd / AddMul / SubMul / DivMul / ElementwiseChain / Gelu
//            weight zero-point folding; Reshape / Unsqueeze / Squeeze / Identity outputs
//            alias their input; last use of every tensor
//   compile: upload initializers, pack MatMulInteger weights once (icx_pack_weight)
//   run:     input shape guard, then every planned op on the caller's stream; intermediate
//            tensors come from a size-class pool on hipMalloc and return to it at their
//            last use (stream order makes the reuse safe).  A fused head whose runtime
//            shapes fall outside its kernel runs its member nodes one by one instead.
//            Shape results and the integer arithmetic on them (an exported model's reshape
//            targets, Slice bounds, Expand shapes) are computed on the host and uploaded
//            only where a device op or the caller reads them.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <exception>
#include <map>
#include <set>
#include <sstream>
#include <string>
#include <vector>

#include "icx_common.hpp"
#include "internal.hpp"

namespace {

using icx::set_error;

size_t dtype_size(int dt) {
    switch (dt) {
        case ICX_I8:
        case ICX_U8:
        case ICX_BOOL: return 1;
        case ICX_I64: return 8;
        default: return 4;
    }
}

const char* dtype_name(int dt) {
    switch (dt) {
        case ICX_I8: return "Int8";
        case ICX_U8: return "UInt8";
        case ICX_I32: return "Int32";
        case ICX_F32: return "Float32";
        case ICX_I64: return "Int64";
        case ICX_BOOL: return "Bool";
        default: return "?";
    }
}

int64_t numel(const std::vector<int64_t>& s) {
    int64_t n = 1;
    for (int64_t d : s) n *= d;
    return n;
}

std::string shape_str(const std::vector<int64_t>& s) {
    std::ostringstream o;
    o << "[";
    for (size_t i = 0; i < s.size(); ++i) o << (i ? ", " : "") << s[i];
    o << "]";
    return o.str();
}

struct HostTensor {
    int dtype = ICX_F32;
    std::vector<int64_t> shape;
    std::vector<uint8_t> data;
    bool all_zero() const {
        for (uint8_t b : data)
            if (b) return false;
        return true;
    }
};

struct Node {
    std::string name, op;
    std::vector<std::string> in, out;
    std::map<std::string, int64_t> attr;
    std::map<std::string, double> fattr;
    std::map<std::string, std::vector<int64_t>> iattrs;
    int64_t attr_or(const std::string& k, int64_t d) const {
        auto it = attr.find(k);
        return it == attr.end() ? d : it->second;
    }
    double fattr_or(const std::string& k, double d) const {
        auto it = fattr.find(k);
        return it == fattr.end() ? d : it->second;
    }
};

// One step of an elementwise chain: v = v op operand (or operand op v).  The operand is a
// tensor, or the product of two (a folded Mul(x_scale, w_scale) node); operand-free steps
// (erf, save, multiply by the saved value) leave it empty.
struct Step {
    int op = ICX_OP_MUL;
    bool lhs = false;
    std::string opnd0, opnd1;
};

enum class Kind { Regular, FusedHead, Skip };
enum class Pattern {
    None,
    QuantizedLinear,
    MulAdd,
    AddMul,
    SubMul,
    DivMul,
    ElementwiseChain,
    Gelu,
    Attention,
    AddLayerNorm,
    DecomposedLayerNorm,
    GatherDequantize
};

const char* kind_name(Kind k) {
    return k == Kind::Regular ? "Regular" : k == Kind::FusedHead ? "FusedHead" : "Skip";
}

const char* pattern_name(Pattern p) {
    switch (p) {
        case Pattern::QuantizedLinear: return "QuantizedLinear";
        case Pattern::MulAdd: return "MulAdd";
        case Pattern::AddMul: return "AddMul";
        case Pattern::SubMul: return "SubMul";
        case Pattern::DivMul: return "DivMul";
        case Pattern::ElementwiseChain: return "ElementwiseChain";
        case Pattern::Gelu: return "Gelu";
        case Pattern::Attention: return "Attention";
        case Pattern::AddLayerNorm: return "AddLayerNorm";
        case Pattern::DecomposedLayerNorm: return "DecomposedLayerNorm";
        case Pattern::GatherDequantize: return "GatherDequantize";
        default: return "-";
    }
}

// One entry of the execution plan (the reference's PlannedOp, src/ir/plan.rs).
struct PlannedOp {
    Node node;
    Kind kind = Kind::Regular;
    Pattern pattern = Pattern::None;
    std::string a, w, a_zp, w_zp;  // QuantizedLinear: the MatMulInteger operands (GatherDequantize:
                                   // indices, table, -, zero point)
    std::string w_scale;           // GatherDequantize: the per-tensor scale
    bool w_zp_folded = false;      // all-zero weight zero point dropped
    std::string chain_in, out;     // chain input (elementwise heads) and fused output
    std::vector<Step> steps;
    std::vector<Node> members;     // nodes folded into this head, in graph order
    std::vector<Node> sub;         // Attention: every node of the pattern, in graph order
    // Attention: q, k, v activations [B, S, H*D]; heads, head size; scale and where it acts
    std::string q, k, v;
    int64_t heads = 0, head_dim = 0;
    float scale = 1.0f;
    bool scale_div = false, scale_q = false;
    std::string q_shape, k_shape, v_shape, o_shape;  // Reshape targets (initializers, or computed at run)
    std::string mask;        // padding mask (Where before the Softmax) broadcasting as [B, 1, 1, S], or ""
    std::string mask_shape;  // the absorbed Expand's target when not the scores' own Shape, or ""
    float fill = 0.0f;       // the score a masked key takes
    // AddLayerNorm, DecomposedLayerNorm: LN(x + res); the decomposed form may lack scale / bias
    std::string ln_x, ln_res, ln_scale, ln_bias;
    float eps = 1e-5f;
    // QuantizedLinear sibling group (heads over one activation, e.g. Q / K / V): the first
    // in plan order (the lead) runs every member's GEMM as one launch over the
    // column-concatenated weight; the other members run nothing.
    std::string group;              // lead's node name, on every member; empty: no group
    std::vector<int> group_members; // lead: plan indices of all members, lead first
    std::string group_w;            // lead: key of the concatenated packed weight
    std::vector<Step> group_steps;  // lead: the chain over the concatenated columns
};

struct DevTensor {
    void* ptr = nullptr;
    int dtype = ICX_F32;
    std::vector<int64_t> shape;
    size_t bytes = 0;
    size_t cls = 0;       // pool size class (pooled tensors)
    bool pooled = false;  // returned to the pool at its last use
};

struct BoundInput {
    int dtype = ICX_F32;
    std::vector<int64_t> shape;
    std::vector<uint8_t> host;  // host data (copied to the device at run)
    const void* dev = nullptr;  // caller's device pointer (used in place)
};

struct PackedW {
    int8_t* packed = nullptr;
    int32_t* colsum = nullptr;
    int dtype = ICX_I8;
    int64_t K = 0, N = 0;
};

// Size-class pool on hipMalloc: power-of-two classes from 256 B.  Reused buffers are not
// cleared (the reference pool zero-fills, src/cuda/memory_pool.rs); every kernel here
// writes its whole output.
class Pool {
   public:
    ~Pool() { release_all(); }
    void* get(size_t bytes, size_t* cls_out) {
        *cls_out = 0;
        if (bytes > (SIZE_MAX >> 1) + 1) return nullptr;  // no power-of-two class holds it
        size_t c = 256;
        while (c < bytes) c <<= 1;
        *cls_out = c;
        auto& fl = free_[c];
        if (!fl.empty()) {
            void* p = fl.back();
            fl.pop_back();
            ++hits_;
            return p;
        }
        void* p = nullptr;
        if (hipMalloc(&p, c) != hipSuccess) return nullptr;
        ++mallocs_;
        held_ += (int64_t)c;
        all_.push_back(p);
        return p;
    }
    void put(void* p, size_t cls) {
        if (p) free_[cls].push_back(p);
    }
    void release_all() {
        for (void* p : all_) (void)hipFree(p);
        all_.clear();
        free_.clear();
        held_ = 0;
    }
    int64_t mallocs_ = 0, hits_ = 0, held_ = 0;

   private:
    std::map<size_t, std::vector<void*>> free_;
    std::vector<void*> all_;
};

}  // namespace

struct icx_graph {
    std::vector<std::pair<std::string, std::vector<int64_t>>> inputs;  // -1 = dynamic dim
    std::map<std::string, HostTensor> inits;
    std::vector<Node> nodes;
    std::vector<std::string> outputs;

    // plan
    bool planned = false, compiled = false;
    bool quant_out_on = true;  // option "quantized_outputs"
    bool qin_on = true;        // option "quantized_inputs" (with quantized_outputs)
    std::vector<PlannedOp> plan;
    std::vector<std::string> live_outputs;     // requested outputs, or the sinks
    std::set<std::string> keep;                // tensors that stay until the next run
    std::map<std::string, size_t> last_use;    // tensor -> plan index of its last reader
    std::set<std::string> rowsum_wanted;       // DQL outputs whose row sums a GEMM reads
    std::set<std::string> range_wanted;        // DQL inputs whose producer leaves their range
    // head output -> the DynamicQuantizeLinear that is its only reader, whose outputs the
    // head's kernel writes itself when the shape allows (the f32 output is never formed): a
    // quantized linear's GEMM (icx::qlinear_dql) or an attention (icx::attention_dql)
    std::map<std::string, Node> quant_out;
    // quantized-linear head output -> the DynamicQuantizeLinear whose outputs only that head
    // reads: the head's launch runs the DQL too (icx::dql_qlinear); the DQL's own plan entry
    // does nothing (names in qin_dql)
    std::map<std::string, Node> qin;
    std::set<std::string> qin_dql;

    // device state
    std::map<std::string, DevTensor> weights;      // uploaded initializers
    std::map<std::string, PackedW> packed;         // packed MatMulInteger weights
    std::map<std::string, BoundInput> bound;       // inputs for the next run
    std::map<std::string, DevTensor> values;       // tensors of the current / last run
    std::map<std::string, HostTensor> hv;          // tensors of this run known on the host
    std::map<std::string, std::string> rowsum_of;  // DQL y -> its row-sum tensor
    std::map<std::string, std::pair<std::string, int>> range_of;  // DQL x -> (partials tensor, count)
    std::set<std::string> dql_done;  // DQL outputs already written by their producer's GEMM
    int64_t quant_fused = 0;         // head launches that quantized their own output
    int64_t qin_fused = 0;           // head launches that ran their input's DQL too
    int64_t dql_single = 0;          // DynamicQuantizeLinear runs done as one launch
    unsigned* qsync = nullptr;       // range-exchange buffer of every launch that uses one (zeroed once)
    hipStream_t last_stream = nullptr;
    bool ran = false;
    Pool pool;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    // a captured run (icx_graph_capture): the HIP graph, its executable form and the output
    // tensors it writes
    hipGraph_t hip_graph = nullptr;
    hipGraphExec_t hip_exec = nullptr;
    std::map<std::string, DevTensor> captured_values;
    std::vector<hipEvent_t> prof_events;  // icx_graph_run_profiled's events, created once

    ~icx_graph() {
        if (ran && last_stream) (void)hipStreamSynchronize(last_stream);
        drop_capture();
        clear_run();
        free_weights();
        for (hipEvent_t e : prof_events) (void)hipEventDestroy(e);
    }
    void drop_capture() {
        if (hip_exec) (void)hipGraphExecDestroy(hip_exec);
        if (hip_graph) (void)hipGraphDestroy(hip_graph);
        hip_exec = nullptr;
        hip_graph = nullptr;
        captured_values.clear();
    }
    void free_weights() {
        for (auto& kv : weights) (void)hipFree(kv.second.ptr);
        weights.clear();
        for (auto& kv : packed) {
            (void)hipFree(kv.second.packed);
            (void)hipFree(kv.second.colsum);
        }
        packed.clear();
        if (ws) (void)hipFree(ws);
        ws = nullptr;
        ws_bytes = 0;
        if (qsync) (void)hipFree(qsync);
        qsync = nullptr;
    }
    void clear_run() {
        for (auto& kv : values)
            if (kv.second.pooled) pool.put(kv.second.ptr, kv.second.cls);
        values.clear();
        hv.clear();
        rowsum_of.clear();
        range_of.clear();
        dql_done.clear();
    }
    void invalidate() {
        planned = compiled = false;
        drop_capture();
    }
    Node* find_node(const std::string& name) {
        for (auto& n : nodes)
            if (n.name == name) return &n;
        return nullptr;
    }
};

namespace {

// ---------------------------------------------------------------------------------------
// planning (host only)
// ---------------------------------------------------------------------------------------
struct GraphIndex {
    std::map<std::string, int> producer;                // tensor -> node index
    std::map<std::string, std::vector<int>> consumers;  // tensor -> node indices
    explicit GraphIndex(const std::vector<Node>& nodes) {
        for (int i = 0; i < (int)nodes.size(); ++i) {
            for (auto& o : nodes[i].out)
                if (!o.empty()) producer[o] = i;
            for (auto& x : nodes[i].in)
                if (!x.empty()) consumers[x].push_back(i);
        }
    }
};

// Ops whose output, for a device tensor, names the input's buffer with another shape.
bool is_view(const std::string& op) {
    return op == "Reshape" || op == "Unsqueeze" || op == "Squeeze" || op == "Identity";
}

int op_code(const std::string& op) {
    if (op == "Add") return ICX_OP_ADD;
    if (op == "Sub") return ICX_OP_SUB;
    if (op == "Mul") return ICX_OP_MUL;
    if (op == "Div") return ICX_OP_DIV;
    return -1;
}

class Planner {
   public:
    explicit Planner(icx_graph& g) : g_(g), gi_(g.nodes) {}

    int run() {
        choose_outputs();
        nodes_ = live_nodes();
        int rc = topo_sort();
        if (rc) return rc;
        merge_duplicates();
        gi_ = GraphIndex(nodes_);
        outs_.clear();
        outs_.insert(g_.live_outputs.begin(), g_.live_outputs.end());
        const int n = (int)nodes_.size();
        std::vector<PlannedOp> ops(n);
        for (int i = 0; i < n; ++i) ops[i].node = nodes_[i];
        // attention first (it owns Transposes / MatMuls), then the quantized linears (they
        // own their Cast / Mul / Add / chain / GELU nodes), residual norms, plain chains
        for (int pass = 0; pass < 4; ++pass) {
            for (int i = 0; i < n; ++i) {
                if (claimed_.count(i)) continue;
                PlannedOp head;
                head.node = nodes_[i];
                std::vector<int> mem;
                bool hit = false;
                switch (pass) {
                    case 0: hit = match_attention(i, head, mem); break;
                    case 1: hit = match_qlinear(i, head, mem); break;
                    case 2: hit = match_add_layer_norm(i, head, mem) || match_layer_norm_chain(i, head, mem); break;
                    default: hit = match_gather_dequant(i, head, mem) || match_chain(i, head, mem); break;
                }
                if (!hit) continue;
                // The head runs at its last member's position: every operand of every member
                // is produced before that point, and nothing else reads the members' outputs.
                int pos = i;
                claimed_.insert(i);
                std::sort(mem.begin(), mem.end());
                for (int m : mem) {
                    claimed_.insert(m);
                    pos = std::max(pos, m);
                    head.members.push_back(nodes_[m]);
                    ops[m].kind = Kind::Skip;
                }
                ops[i].kind = Kind::Skip;
                if (head.pattern == Pattern::Attention || head.pattern == Pattern::GatherDequantize) {
                    std::vector<int> all = mem;
                    all.push_back(i);
                    std::sort(all.begin(), all.end());
                    for (int k : all) head.sub.push_back(nodes_[k]);
                }
                ops[pos] = head;
            }
        }
        g_.plan = ops;
        group_siblings();
        g_.rowsum_wanted.clear();
        for (auto& op : g_.plan) {
            if (op.pattern != Pattern::QuantizedLinear) continue;
            const bool u8w = g_.inits[op.w].dtype == ICX_U8;
            if (!u8w && (op.w_zp.empty() || op.w_zp_folded)) continue;
            auto p = gi_.producer.find(op.a);
            if (p != gi_.producer.end() && nodes_[p->second].op == "DynamicQuantizeLinear")
                g_.rowsum_wanted.insert(op.a);
        }
        // a DynamicQuantizeLinear whose input is the output of a LayerNorm, attention or
        // quantized-linear head takes that input's range from the head's kernel and runs its
        // quantize launch only
        g_.range_wanted.clear();
        {
            std::set<std::string> heads_out;
            for (auto& op : g_.plan)
                if (op.kind == Kind::FusedHead && op.group.empty() &&
                    (op.pattern == Pattern::AddLayerNorm || op.pattern == Pattern::DecomposedLayerNorm ||
                     op.pattern == Pattern::Attention ||
                     op.pattern == Pattern::QuantizedLinear))
                    heads_out.insert(op.out);
            for (auto& op : g_.plan)
                if (op.kind == Kind::Regular && op.node.op == "DynamicQuantizeLinear" && op.node.in.size() == 1 &&
                    heads_out.count(op.node.in[0]))
                    g_.range_wanted.insert(op.node.in[0]);
        }
        // last readers; a view's output (Reshape, Unsqueeze, ...) aliases its input's buffer, so uses of the alias
        // extend the buffer's life, and a live alias keeps it until the next run
        g_.last_use.clear();
        std::map<std::string, std::string> root;
        auto root_of = [&](const std::string& t) {
            auto it = root.find(t);
            return it == root.end() ? t : it->second;
        };
        for (size_t i = 0; i < g_.plan.size(); ++i) {
            const PlannedOp& op = g_.plan[i];
            if (op.kind == Kind::Skip) continue;
            std::vector<std::string> uses = op.node.in;
            for (auto& st : op.steps) {
                uses.push_back(st.opnd0);
                if (!st.opnd1.empty()) uses.push_back(st.opnd1);
            }
            if (op.kind == Kind::FusedHead)
                for (auto& m : op.members) uses.insert(uses.end(), m.in.begin(), m.in.end());
            for (auto& x : {op.chain_in, op.q, op.k, op.v, op.ln_x, op.ln_res, op.a}) uses.push_back(x);
            for (auto& u : uses)
                if (!u.empty()) {
                    g_.last_use[u] = i;
                    g_.last_use[root_of(u)] = i;
                }
            if (op.kind == Kind::Regular && is_view(op.node.op) && !op.node.out.empty() && !op.node.in.empty())
                root[op.node.out[0]] = root_of(op.node.in[0]);
            for (auto& m : op.sub)  // a fused head run node by node creates the same aliases
                if (is_view(m.op) && !m.out.empty()) root[m.out[0]] = root_of(m.in[0]);
        }
        g_.keep.clear();
        for (auto& o : g_.live_outputs) {
            g_.keep.insert(o);
            g_.keep.insert(root_of(o));
        }
        // a quantized-linear head (Int8 weight without zero point, no sibling group) or an
        // attention head whose output only a DynamicQuantizeLinear reads, and whose quantized
        // output no GEMM reads row sums of: the head's kernel may write the DQL's outputs itself
        g_.quant_out.clear();
        for (auto& op : g_.plan) {
            if (op.kind != Kind::FusedHead || !g_.quant_out_on) continue;
            if (op.pattern == Pattern::QuantizedLinear) {
                if (!op.group.empty()) continue;
                if (g_.inits[op.w].dtype != ICX_I8 || !(op.w_zp.empty() || op.w_zp_folded)) continue;
            } else if (op.pattern != Pattern::Attention) {
                continue;
            }
            if (g_.keep.count(op.out) || !g_.range_wanted.count(op.out)) continue;
            auto cs = gi_.consumers.find(op.out);
            if (cs == gi_.consumers.end() || cs->second.size() != 1) continue;
            const Node& d = nodes_[cs->second[0]];
            if (d.op != "DynamicQuantizeLinear" || d.in.size() != 1 || d.out.size() != 3) continue;
            if (g_.rowsum_wanted.count(d.out[0])) continue;
            g_.quant_out[op.out] = d;
        }
        // a DynamicQuantizeLinear whose outputs only one quantized-linear head reads (Int8
        // weight without zero point, no sibling group, f32 output) and whose input no head
        // leaves the range of: the head's GEMM launch runs the DQL too
        g_.qin.clear();
        g_.qin_dql.clear();
        for (size_t i = 0; i < g_.plan.size() && g_.quant_out_on && g_.qin_on; ++i) {
            const PlannedOp& op = g_.plan[i];
            if (op.kind != Kind::FusedHead || op.pattern != Pattern::QuantizedLinear || !op.group.empty()) continue;
            if (g_.inits[op.w].dtype != ICX_I8 || !(op.w_zp.empty() || op.w_zp_folded)) continue;
            if (g_.quant_out.count(op.out)) continue;
            auto pr = gi_.producer.find(op.a);
            if (pr == gi_.producer.end()) continue;
            const Node& d = nodes_[pr->second];
            if (d.op != "DynamicQuantizeLinear" || d.in.size() != 1 || d.out.size() != 3 || op.a_zp != d.out[2])
                continue;
            if (g_.range_wanted.count(d.in[0]) || g_.rowsum_wanted.count(d.out[0])) continue;
            if (g_.quant_out.count(d.in[0])) continue;  // its producer writes this DQL's outputs itself
            std::set<std::string> mine = {op.node.name};
            for (auto& m : op.members) mine.insert(m.name);
            bool only = true;
            for (auto& o : d.out) {
                auto cs = gi_.consumers.find(o);
                if (cs == gi_.consumers.end()) continue;
                for (int c : cs->second) only = only && mine.count(nodes_[c].name) > 0;
            }
            bool regular = false;  // the DQL runs as a plan entry of its own (before the head)
            for (size_t j = 0; j < i; ++j)
                regular = regular || (g_.plan[j].kind == Kind::Regular && g_.plan[j].node.name == d.name);
            if (!only || !regular) continue;
            g_.qin[op.out] = d;
            g_.qin_dql.insert(d.name);
            // the DQL's input is read at the head now: keep its buffer until then
            for (auto& x : {d.in[0], root_of(d.in[0])})
                if (g_.last_use[x] < i) g_.last_use[x] = i;
        }
        g_.planned = true;
        return ICX_OK;
    }

   private:
    // Shape / mask plumbing nodes with the same op, inputs and attributes compute the same
    // outputs: keep the first, point the readers of the others at its outputs (an export
    // recomputes the padding mask's Equal(mask, 0) in every layer).  Only those ops: a shared
    // node of a fusion pattern (the x_scale * w_scale Mul of Q, K and V, say) would stop the
    // pattern from owning it.  A node whose output the caller asked for stays.  Runs on the
    // topologically sorted list, so the kept node precedes every reader of the ones it replaces.
    static bool mergeable(const std::string& op) {
        return op == "Shape" || op == "Equal" || op == "Cast" || op == "Slice" || op == "Concat" ||
               op == "Unsqueeze" || op == "Squeeze" || op == "Gather" || op == "Expand" || op == "Where";
    }
    void merge_duplicates() {
        std::map<std::string, std::string> rename;
        std::map<std::string, size_t> seen;
        std::set<std::string> live(g_.live_outputs.begin(), g_.live_outputs.end());
        std::vector<Node> kept;
        for (Node n : nodes_) {
            for (auto& i : n.in) {
                auto r = rename.find(i);
                if (r != rename.end()) i = r->second;
            }
            std::ostringstream key;
            key << n.op << '\x1f' << n.in.size() << '\x1f' << n.out.size();
            for (auto& i : n.in) {  // a small initializer by its value (exports repeat constants)
                auto it = g_.inits.find(i);
                if (it != g_.inits.end() && it->second.data.size() <= 64) {
                    key << "\x1f#" << it->second.dtype << shape_str(it->second.shape);
                    for (uint8_t b : it->second.data) key << '.' << (int)b;
                } else {
                    key << '\x1f' << i;
                }
            }
            for (auto& a : n.attr) key << '\x1e' << a.first << '=' << a.second;
            for (auto& a : n.fattr) {
                uint64_t b;
                std::memcpy(&b, &a.second, 8);
                key << '\x1d' << a.first << '=' << b;
            }
            for (auto& a : n.iattrs) {
                key << '\x1c' << a.first << '=';
                for (int64_t v : a.second) key << v << ',';
            }
            bool is_live = !mergeable(n.op);
            for (auto& o : n.out) is_live = is_live || live.count(o);
            auto it = seen.find(key.str());
            bool same_outs = it != seen.end();
            for (size_t j = 0; same_outs && j < n.out.size(); ++j)
                same_outs = n.out[j].empty() || !kept[it->second].out[j].empty();
            if (same_outs && !is_live) {
                const Node& k = kept[it->second];
                for (size_t j = 0; j < n.out.size(); ++j)
                    if (!n.out[j].empty()) rename[n.out[j]] = k.out[j];
                continue;
            }
            if (it == seen.end()) seen[key.str()] = kept.size();
            kept.push_back(std::move(n));
        }
        nodes_ = std::move(kept);
    }

    icx_graph& g_;
    GraphIndex gi_;
    std::vector<Node> nodes_;
    std::set<std::string> outs_;
    std::set<int> claimed_;

    // ---- sibling quantized linears -------------------------------------------------------
    // Heads that read the same activation and zero point, with weights of one dtype and
    // shape [K, Nh] (Nh a multiple of 256), no weight zero point (absent or all zero), and
    // chains of the same steps whose operands are either one shared scalar or static f32
    // scalars / [Nh] vectors, become one GEMM over the concatenated [K, n*Nh] weight with
    // each head's operands concatenated into [n*Nh] column vectors.  Every column then
    // goes through exactly the arithmetic of its own head: a product operand is still
    // p0 * p1 rounded once, and a scalar expanded to a column is the same value.
    bool scalar_tensor(const std::string& t) const {
        auto it = g_.inits.find(t);
        if (it != g_.inits.end()) return it->second.dtype == ICX_F32 && numel(it->second.shape) == 1;
        const int p = producer(t);  // y_scale of a DynamicQuantizeLinear is a scalar
        return p >= 0 && nodes_[p].op == "DynamicQuantizeLinear" && nodes_[p].out.size() > 1 && nodes_[p].out[1] == t;
    }
    bool column_init(const std::string& t, int64_t nh) const {
        auto it = g_.inits.find(t);
        if (it == g_.inits.end() || it->second.dtype != ICX_F32) return false;
        const auto& sh = it->second.shape;
        return numel(sh) == 1 || (!sh.empty() && sh.back() == nh && numel(sh) == nh);
    }
    // operand slot shared by name (a scalar) or concatenable across the heads
    bool groupable_operand(const std::vector<const PlannedOp*>& hs, size_t k, int which, int64_t nh) const {
        auto name = [&](const PlannedOp* h) { return which ? h->steps[k].opnd1 : h->steps[k].opnd0; };
        const std::string first = name(hs[0]);
        bool same = true;
        for (auto* h : hs) same = same && name(h) == first;
        if (same) return first.empty() || scalar_tensor(first);
        for (auto* h : hs)
            if (name(h).empty() || !column_init(name(h), nh)) return false;
        return true;
    }
    bool siblings(const PlannedOp& a, const PlannedOp& b) const {
        if (a.a != b.a || a.a_zp != b.a_zp || a.steps.size() != b.steps.size()) return false;
        const HostTensor& wa = g_.inits.at(a.w);
        const HostTensor& wb = g_.inits.at(b.w);
        if (wa.dtype != wb.dtype || wa.shape != wb.shape) return false;
        for (size_t k = 0; k < a.steps.size(); ++k)
            if (a.steps[k].op != b.steps[k].op || a.steps[k].lhs != b.steps[k].lhs ||
                a.steps[k].opnd1.empty() != b.steps[k].opnd1.empty())
                return false;
        return true;
    }
    void group_siblings() {
        std::vector<PlannedOp>& plan = g_.plan;
        auto candidate = [&](const PlannedOp& op) {
            if (op.kind != Kind::FusedHead || op.pattern != Pattern::QuantizedLinear || !op.group.empty()) return false;
            const HostTensor& w = g_.inits.at(op.w);
            return (op.w_zp.empty() || op.w_zp_folded) && w.shape.size() == 2 && w.shape[1] % 256 == 0 &&
                   w.shape[1] > 0;
        };
        for (size_t i = 0; i < plan.size(); ++i) {
            if (!candidate(plan[i])) continue;
            std::vector<int> idx = {(int)i};
            for (size_t j = i + 1; j < plan.size() && idx.size() < (size_t)icx::kMaxSegments; ++j)
                if (candidate(plan[j]) && siblings(plan[i], plan[j])) idx.push_back((int)j);
            if (idx.size() < 2) continue;
            std::vector<const PlannedOp*> hs;
            for (int k : idx) hs.push_back(&plan[k]);
            const int64_t nh = g_.inits.at(plan[i].w).shape[1];
            bool ok = true;
            for (size_t k = 0; ok && k < plan[i].steps.size(); ++k) {
                if (plan[i].steps[k].op > ICX_OP_DIV) continue;  // operand-free step
                ok = groupable_operand(hs, k, 0, nh) && groupable_operand(hs, k, 1, nh);
            }
            if (!ok) continue;
            PlannedOp& lead = plan[i];
            lead.group_members = idx;
            lead.group_w = lead.out + "::group.w";
            lead.group_steps = lead.steps;
            for (size_t k = 0; k < lead.steps.size(); ++k) {
                if (lead.steps[k].op > ICX_OP_DIV) continue;
                for (int which = 0; which < 2; ++which) {
                    std::string& nm = which ? lead.group_steps[k].opnd1 : lead.group_steps[k].opnd0;
                    bool same = true;
                    for (auto* h : hs) same = same && (which ? h->steps[k].opnd1 : h->steps[k].opnd0) == nm;
                    if (!same) nm = lead.out + "::group.c" + std::to_string(k) + "." + std::to_string(which);
                }
            }
            for (int k : idx) plan[k].group = lead.node.name;
        }
    }

    // Requested outputs, or every node output that no node reads (mod.rs:505-519).
    void choose_outputs() {
        g_.live_outputs = g_.outputs;
        if (!g_.live_outputs.empty()) return;
        for (auto& n : g_.nodes)
            for (auto& o : n.out)
                if (!o.empty() && !gi_.consumers.count(o)) g_.live_outputs.push_back(o);
    }
    // Nodes that contribute to a live output (dead-node elimination), to a fixed point:
    // node order is arbitrary before sorting.
    std::vector<Node> live_nodes() const {
        std::set<std::string> need(g_.live_outputs.begin(), g_.live_outputs.end());
        std::vector<bool> keep(g_.nodes.size(), false);
        bool changed = true;
        while (changed) {
            changed = false;
            for (size_t i = 0; i < g_.nodes.size(); ++i) {
                if (keep[i]) continue;
                bool live = false;
                for (auto& o : g_.nodes[i].out) live = live || (!o.empty() && need.count(o));
                if (!live) continue;
                keep[i] = true;
                changed = true;
                for (auto& x : g_.nodes[i].in)
                    if (!x.empty()) need.insert(x);
            }
        }
        std::vector<Node> out;
        for (size_t i = 0; i < g_.nodes.size(); ++i)
            if (keep[i]) out.push_back(g_.nodes[i]);
        return out;
    }
    // Kahn's algorithm, keeping insertion order among ready nodes.
    int topo_sort() {
        GraphIndex gi(nodes_);
        std::vector<int> indeg(nodes_.size(), 0);
        for (size_t i = 0; i < nodes_.size(); ++i)
            for (auto& x : nodes_[i].in)
                if (!x.empty() && gi.producer.count(x)) ++indeg[i];
        std::vector<Node> sorted;
        std::vector<bool> done(nodes_.size(), false);
        while (sorted.size() < nodes_.size()) {
            bool progressed = false;
            for (size_t i = 0; i < nodes_.size(); ++i) {
                if (done[i] || indeg[i]) continue;
                done[i] = true;
                progressed = true;
                sorted.push_back(nodes_[i]);
                for (auto& o : nodes_[i].out) {
                    auto c = gi.consumers.find(o);
                    if (c != gi.consumers.end())
                        for (int k : c->second) --indeg[k];
                }
            }
            if (!progressed) {
                set_error("graph has a cycle");
                return ICX_ERR_INVALID_ARG;
            }
        }
        nodes_.swap(sorted);
        return ICX_OK;
    }

    bool is_init(const std::string& t) const { return g_.inits.count(t) > 0; }
    bool static_f32(const std::string& t) const {
        auto it = g_.inits.find(t);
        return it != g_.inits.end() && it->second.dtype == ICX_F32;
    }
    bool static_scalar(const std::string& t, float* v) const {
        auto it = g_.inits.find(t);
        if (it == g_.inits.end() || it->second.dtype != ICX_F32 || numel(it->second.shape) != 1) return false;
        std::memcpy(v, it->second.data.data(), 4);
        return true;
    }
    int producer(const std::string& t) const {
        auto it = gi_.producer.find(t);
        return it == gi_.producer.end() ? -1 : it->second;
    }
    // The single reader of t, or -1 (also when t is a live output: it must materialise).
    int sole_consumer(const std::string& t) const {
        if (outs_.count(t)) return -1;
        auto it = gi_.consumers.find(t);
        if (it == gi_.consumers.end() || it->second.size() != 1) return -1;
        return it->second[0];
    }
    bool is_op(int i, const char* op) const { return i >= 0 && !claimed_.count(i) && nodes_[i].op == op; }
    bool has_perm(int i, std::initializer_list<int64_t> perm) const {
        auto it = nodes_[i].iattrs.find("perm");
        return it != nodes_[i].iattrs.end() && it->second == std::vector<int64_t>(perm);
    }

    // Node ni as a chain step over `cur` with a static f32 operand.
    bool as_step(int ni, const std::string& cur, Step& st) const {
        const Node& n = nodes_[ni];
        if (op_code(n.op) < 0 || n.in.size() != 2 || n.out.size() != 1 || claimed_.count(ni)) return false;
        const bool left = n.in[0] == cur, right = n.in[1] == cur;
        if (left == right) return false;
        const std::string& other = left ? n.in[1] : n.in[0];
        if (!static_f32(other)) return false;
        st.op = op_code(n.op);
        st.lhs = !left;
        st.opnd0 = other;
        st.opnd1.clear();
        return true;
    }
    // x -> [Div(x, c0) -> Erf -> Add(., c1)] -> Mul(x, .) [-> Mul(., c2)]: the erf-GELU of
    // PyTorch's export.  Appends SAVE, DIV, ERF, ADD, MUL_SAVED [, MUL] to `steps`.
    bool match_gelu(std::string& cur, std::vector<Step>& steps, std::vector<int>& mem) const {
        if (outs_.count(cur)) return false;
        auto cs = gi_.consumers.find(cur);
        if (cs == gi_.consumers.end() || cs->second.size() != 2) return false;
        int di = -1, mi = -1;
        for (int c : cs->second) {
            if (is_op(c, "Div") && nodes_[c].in.size() == 2 && nodes_[c].in[0] == cur) di = c;
            if (is_op(c, "Mul")) mi = c;
        }
        if (di < 0 || mi < 0 || di == mi || !static_f32(nodes_[di].in[1])) return false;
        const int ei = sole_consumer(nodes_[di].out[0]);
        if (!is_op(ei, "Erf")) return false;
        const int ai = sole_consumer(nodes_[ei].out[0]);
        Step add;
        if (ai < 0 || !as_step(ai, nodes_[ei].out[0], add) || add.op != ICX_OP_ADD) return false;
        const std::string a_out = nodes_[ai].out[0];
        if (sole_consumer(a_out) != mi) return false;
        const Node& m = nodes_[mi];
        if (m.in.size() != 2 || !((m.in[0] == cur && m.in[1] == a_out) || (m.in[1] == cur && m.in[0] == a_out)))
            return false;
        const size_t need = steps.size() + 5;
        if (need > ICX_MAX_CHAIN) return false;
        Step sv, dv, ev, ms;
        sv.op = ICX_OP_SAVE;
        dv.op = ICX_OP_DIV;
        dv.opnd0 = nodes_[di].in[1];
        ev.op = ICX_OP_ERF;
        ms.op = ICX_OP_MUL_SAVED;
        steps.insert(steps.end(), {sv, dv, ev, add, ms});
        mem.insert(mem.end(), {di, ei, ai, mi});
        cur = m.out[0];
        const int hi = sole_consumer(cur);
        Step half;
        if (steps.size() < ICX_MAX_CHAIN && hi >= 0 && as_step(hi, cur, half) && half.op == ICX_OP_MUL) {
            steps.push_back(half);
            mem.push_back(hi);
            cur = nodes_[hi].out[0];
        }
        return true;
    }
    void extend_chain(std::string& cur, std::vector<Step>& steps, std::vector<int>& mem) const {
        while ((int)steps.size() < ICX_MAX_CHAIN) {
            const int c = sole_consumer(cur);
            Step st;
            if (c >= 0 && as_step(c, cur, st)) {
                steps.push_back(st);
                mem.push_back(c);
                cur = nodes_[c].out[0];
                continue;
            }
            if (!match_gelu(cur, steps, mem)) break;
        }
    }

    // MatMulInteger(A, W initializer [K,N]) -> Cast(to=FLOAT) -> Mul(scale) [-> chain]
    bool match_qlinear(int mi, PlannedOp& head, std::vector<int>& mem) {
        const Node& m = nodes_[mi];
        if (m.op != "MatMulInteger" || m.in.size() < 2 || m.in.size() > 4 || m.out.size() != 1) return false;
        auto wi = g_.inits.find(m.in[1]);
        if (wi == g_.inits.end() || wi->second.shape.size() != 2) return false;
        if (wi->second.dtype != ICX_I8 && wi->second.dtype != ICX_U8) return false;
        const std::string a_zp = m.in.size() > 2 ? m.in[2] : "";
        const std::string w_zp = m.in.size() > 3 ? m.in[3] : "";
        if (!w_zp.empty() && !is_init(w_zp)) return false;
        const int ci = sole_consumer(m.out[0]);
        if (is_op(ci, "DequantizeLinear")) return match_dequant_head(mi, ci, head, mem);
        if (!is_op(ci, "Cast") || nodes_[ci].attr_or("to", -1) != 1 || nodes_[ci].out.size() != 1) return false;
        const std::string cast_out = nodes_[ci].out[0];
        const int si = sole_consumer(cast_out);
        if (!is_op(si, "Mul") || nodes_[si].in.size() != 2 || nodes_[si].out.size() != 1) return false;
        const Node& s1 = nodes_[si];
        const bool left = s1.in[0] == cast_out, right = s1.in[1] == cast_out;
        if (left == right) return false;
        const std::string scale = left ? s1.in[1] : s1.in[0];
        Step st;
        st.op = ICX_OP_MUL;
        st.lhs = !left;
        mem = {ci, si};
        // scale = Mul(x_scale, w_scale) read only here: a product operand, rounded once
        const int sp = producer(scale);
        if (is_op(sp, "Mul") && nodes_[sp].in.size() == 2 && sole_consumer(scale) == si) {
            st.opnd0 = nodes_[sp].in[0];
            st.opnd1 = nodes_[sp].in[1];
            mem.push_back(sp);
        } else {
            st.opnd0 = scale;
        }
        head.steps = {st};
        std::string cur = s1.out[0];
        extend_chain(cur, head.steps, mem);
        head.kind = Kind::FusedHead;
        head.pattern = Pattern::QuantizedLinear;
        head.a = m.in[0];
        head.w = m.in[1];
        head.a_zp = a_zp;
        head.w_zp = w_zp;
        head.out = cur;
        // zero-point folding: an all-zero weight zero point contributes nothing
        head.w_zp_folded = !w_zp.empty() && g_.inits[w_zp].all_zero();
        return true;
    }

    // MatMulInteger(A, W) -> DequantizeLinear(acc, scale, [zp]) [-> chain]: the int32
    // DequantizeLinear of the CPU forward, (acc as f32 - zp as f32) * scale
    // (src/operators/dequantize_linear.rs:158-174), as the chain steps Sub(zp as f32),
    // Mul(scale) after the GEMM's Cast — each one rounding, as there.  The reference GPU runs it
    // as its own kernel (dequantize_linear_i32_kernel, src/cuda/ops/quantize_kernels.rs:72-81).
    // Needs a static f32 scale and an optional static Int32 zero point, per tensor or per
    // output column (a [N] scale whose axis is the output's last).
    bool match_dequant_head(int mi, int di, PlannedOp& head, std::vector<int>& mem) {
        const Node& m = nodes_[mi];
        const Node& dq = nodes_[di];
        if (dq.in.size() < 2 || dq.in.size() > 3 || dq.out.size() != 1 || dq.in[0] != m.out[0]) return false;
        const int64_t N = g_.inits[m.in[1]].shape[1];
        auto sc = g_.inits.find(dq.in[1]);
        if (sc == g_.inits.end() || sc->second.dtype != ICX_F32) return false;
        const int64_t ns = numel(sc->second.shape);
        if (ns != 1 && !(ns == N && sc->second.shape.size() == 1)) return false;
        if (ns != 1 && N != 1) {  // per axis: the axis must be the output's last
            const int64_t ax = dq.attr_or("axis", 1);
            const int r = rank_of(m.in[0]);
            if (!(ax == -1 || (r > 0 && (ax == r - 1 || ax == -1)))) return false;
            if (ax < -1) return false;
        }
        std::string zpf;
        if (dq.in.size() == 3 && !dq.in[2].empty()) {
            auto zi = g_.inits.find(dq.in[2]);
            if (zi == g_.inits.end() || zi->second.dtype != ICX_I32 || numel(zi->second.shape) != ns) return false;
            if (!zi->second.all_zero()) {
                // the zero point as f32 (x as f32, round to nearest even), a plan-made operand
                HostTensor f;
                f.dtype = ICX_F32;
                f.shape = sc->second.shape;
                f.data.resize(4 * (size_t)ns);
                const int32_t* z = reinterpret_cast<const int32_t*>(zi->second.data.data());
                for (int64_t j = 0; j < ns; ++j) {
                    const float v = (float)z[j];
                    std::memcpy(&f.data[4 * (size_t)j], &v, 4);
                }
                zpf = dq.name + "::zero_point_f32";
                g_.inits[zpf] = f;
            }
        }
        head.steps.clear();
        if (!zpf.empty()) {
            Step sub;
            sub.op = ICX_OP_SUB;
            sub.opnd0 = zpf;
            head.steps.push_back(sub);
        }
        Step mul;
        mul.op = ICX_OP_MUL;
        mul.opnd0 = dq.in[1];
        head.steps.push_back(mul);
        mem = {di};
        std::string cur = dq.out[0];
        extend_chain(cur, head.steps, mem);
        head.kind = Kind::FusedHead;
        head.pattern = Pattern::QuantizedLinear;
        head.a = m.in[0];
        head.w = m.in[1];
        head.a_zp = m.in.size() > 2 ? m.in[2] : "";
        head.w_zp = m.in.size() > 3 ? m.in[3] : "";
        head.out = cur;
        head.w_zp_folded = !head.w_zp.empty() && g_.inits[head.w_zp].all_zero();
        return true;
    }

    // Rank of a tensor from the graph's inputs, initializers and the ops on this path; -1
    // when it cannot be told before a run.
    int rank_of(const std::string& t, int depth = 0) const {
        if (depth > 256) return -1;
        for (auto& in : g_.inputs)
            if (in.first == t) return (int)in.second.size();
        auto it = g_.inits.find(t);
        if (it != g_.inits.end()) return (int)it->second.shape.size();
        const int pi = producer(t);
        if (pi < 0) return -1;
        const Node& n = nodes_[pi];
        const std::string& op = n.op;
        if (op == "DynamicQuantizeLinear") return t == n.out[0] ? rank_of(n.in[0], depth + 1) : 0;
        if (op == "MatMulInteger" || op == "Cast" || op == "Erf" || op == "Softmax" || op == "LayerNormalization" ||
            op == "DequantizeLinear" || op == "Transpose" || op == "Sqrt" || op == "Pow" ||
            (op == "ReduceMean" && n.attr_or("keepdims", 1) != 0 && (n.in.size() > 1 || n.iattrs.count("axes"))))
            return n.in.empty() ? -1 : rank_of(n.in[0], depth + 1);
        if (op == "Reshape" && n.in.size() == 2) {
            auto sh = g_.inits.find(n.in[1]);
            return sh == g_.inits.end() ? -1 : (int)numel(sh->second.shape);
        }
        if (op == "Gather" && n.in.size() == 2) {
            const int rd = rank_of(n.in[0], depth + 1), ri = rank_of(n.in[1], depth + 1);
            return rd < 1 || ri < 0 ? -1 : rd - 1 + ri;
        }
        if ((op_code(op) >= 0 || op == "MatMul") && n.in.size() == 2) {
            const int a = rank_of(n.in[0], depth + 1), b = rank_of(n.in[1], depth + 1);
            return a < 0 || b < 0 ? -1 : std::max(a, b);
        }
        return -1;
    }

    // Two or more binary ops over one running tensor with static operands, or a GELU.
    bool match_chain(int ni, PlannedOp& head, std::vector<int>& mem) {
        const Node& n = nodes_[ni];
        std::vector<Step> steps;
        std::string in, cur;
        mem.clear();
        bool gelu_start = false;
        if (n.op == "Div" && n.in.size() == 2 && !static_f32(n.in[0])) {
            // a GELU whose input is this Div's dividend
            in = cur = n.in[0];
            std::vector<int> gm;
            if (match_gelu(cur, steps, gm) && std::find(gm.begin(), gm.end(), ni) != gm.end()) {
                for (int m : gm)
                    if (m != ni) mem.push_back(m);
                extend_chain(cur, steps, mem);
                gelu_start = true;
            } else {
                steps.clear();
            }
        }
        if (gelu_start) {
        } else if (op_code(n.op) >= 0 && n.in.size() == 2 && n.out.size() == 1) {
            if (static_f32(n.in[1]) && !static_f32(n.in[0])) in = n.in[0];
            else if (static_f32(n.in[0]) && !static_f32(n.in[1])) in = n.in[1];
            else return false;
            Step st;
            if (!as_step(ni, in, st)) return false;
            steps.push_back(st);
            cur = n.out[0];
            extend_chain(cur, steps, mem);
            if (steps.size() < 2) return false;
        } else {
            return false;
        }
        head.kind = Kind::FusedHead;
        head.pattern = Pattern::ElementwiseChain;
        bool gelu = false;
        for (auto& s : steps) gelu = gelu || s.op == ICX_OP_ERF;
        if (gelu) head.pattern = Pattern::Gelu;
        if (steps.size() == 2) {
            const int a = steps[0].op, b = steps[1].op;
            if (a == ICX_OP_MUL && b == ICX_OP_ADD) head.pattern = Pattern::MulAdd;
            if (a == ICX_OP_ADD && b == ICX_OP_MUL) head.pattern = Pattern::AddMul;
            if (a == ICX_OP_SUB && b == ICX_OP_MUL) head.pattern = Pattern::SubMul;
            if (a == ICX_OP_DIV && b == ICX_OP_MUL) head.pattern = Pattern::DivMul;
        }
        head.chain_in = in;
        head.steps = steps;
        head.out = cur;
        return true;
    }

    // LayerNormalization(Add(a, b)) with the Add read only by the norm.
    bool match_add_layer_norm(int li, PlannedOp& head, std::vector<int>& mem) {
        const Node& ln = nodes_[li];
        if (ln.op != "LayerNormalization" || ln.in.size() != 3 || ln.out.empty() || ln.attr_or("axis", -1) != -1)
            return false;
        const int ai = producer(ln.in[0]);
        if (!is_op(ai, "Add") || nodes_[ai].in.size() != 2 || sole_consumer(ln.in[0]) != li) return false;
        head.kind = Kind::FusedHead;
        head.pattern = Pattern::AddLayerNorm;
        head.ln_x = nodes_[ai].in[0];
        head.ln_res = nodes_[ai].in[1];
        head.ln_scale = ln.in[1];
        head.ln_bias = ln.in[2];
        head.eps = (float)ln.fattr_or("epsilon", 1e-5);
        head.out = ln.out[0];
        mem = {ai};
        return true;
    }

    // ReduceMean over the last axis with keepdims: axes [-1] or [rank - 1] from its Int64
    // initializer input (opset 18) or its `axes` attribute (earlier opsets).
    bool last_axis_mean(int i) const {
        const Node& n = nodes_[i];
        if (n.op != "ReduceMean" || n.in.empty() || n.out.size() != 1 || n.attr_or("keepdims", 1) == 0) return false;
        int64_t ax;
        if (n.in.size() > 1 && !n.in[1].empty()) {
            auto it = g_.inits.find(n.in[1]);
            if (it == g_.inits.end() || it->second.dtype != ICX_I64 || numel(it->second.shape) != 1) return false;
            std::memcpy(&ax, it->second.data.data(), 8);
        } else {
            auto it = n.iattrs.find("axes");
            if (it == n.iattrs.end() || it->second.size() != 1) return false;
            ax = it->second[0];
        }
        if (ax == -1) return true;
        const int r = rank_of(n.in[0]);
        return r > 0 && ax == r - 1;
    }
    // The static per-column operand of Mul / Add node k over `cur`: an f32 initializer of
    // shape [.., C] with only ones before C, C >= 2 (checked against the normalised axis at run).
    bool affine_operand(int k, const std::string& cur, std::string* o) const {
        const Node& n = nodes_[k];
        if (n.in.size() != 2 || n.out.size() != 1) return false;
        const bool left = n.in[0] == cur, right = n.in[1] == cur;
        if (left == right) return false;
        const std::string& t = left ? n.in[1] : n.in[0];
        auto it = g_.inits.find(t);
        if (it == g_.inits.end() || it->second.dtype != ICX_F32) return false;
        const auto& sh = it->second.shape;
        if (sh.empty() || sh.back() < 2) return false;
        for (size_t d = 0; d + 1 < sh.size(); ++d)
            if (sh[d] != 1) return false;
        *o = t;
        return true;
    }

    // LayerNorm as an export that decomposes it writes it (PyTorch below opset 17; the
    // reference's DistilBERT-INT8, whose ops include ReduceMean, Pow and Sqrt):
    //     mean = ReduceMean(x); c = Sub(x, mean); v = ReduceMean(Pow(c, 2));
    //     y = Div(c, Sqrt(Add(v, eps))) [-> Mul(., gamma)] [-> Add(., beta)]
    // with both means over the last axis (keepdims), optionally of x = Add(a, b) read by the
    // two only.  Node by node this is exactly the arithmetic of the LayerNormalization kernel,
    // in its order: the means are ndarray's unrolled sums divided by the length
    // (src/operators/reduce_mean.rs:64-72), the square is c * c, then one rounding each for
    // the Add, Sqrt, Div, Mul and Add (src/operators/{sub,pow,add,sqrt,div,mul}.rs) — so the
    // chain runs as one launch of that kernel (icx_layer_norm_f32; no Mul / Add tail: NULL
    // scale / bias).  The reference CPU squares with powf(c, 2), which differs from c * c in
    // the last bit for ~0.07 % of c; the reference GPU fuses only the Add -> Sqrt -> Div tail
    // (DivRsqrt, src/cuda/kernels/fused/mod.rs:131-173).
    bool match_layer_norm_chain(int mi, PlannedOp& head, std::vector<int>& mem) {
        if (!last_axis_mean(mi)) return false;
        const Node& m1 = nodes_[mi];
        const std::string x = m1.in[0], mean = m1.out[0];
        const int si = sole_consumer(mean);
        if (!is_op(si, "Sub") || nodes_[si].in.size() != 2 || nodes_[si].in[0] != x || nodes_[si].in[1] != mean ||
            nodes_[si].out.size() != 1)
            return false;
        const std::string c = nodes_[si].out[0];
        auto cs = gi_.consumers.find(c);
        if (outs_.count(c) || cs == gi_.consumers.end() || cs->second.size() != 2) return false;
        int pi = -1, di = -1;
        for (int k : cs->second) {
            if (is_op(k, "Pow") && nodes_[k].in.size() == 2 && nodes_[k].in[0] == c && nodes_[k].out.size() == 1) pi = k;
            if (is_op(k, "Div") && nodes_[k].in.size() == 2 && nodes_[k].in[0] == c && nodes_[k].out.size() == 1) di = k;
        }
        float ex;
        if (pi < 0 || di < 0 || !static_scalar(nodes_[pi].in[1], &ex) || ex != 2.0f) return false;
        const std::string sq = nodes_[pi].out[0];
        const int m2 = sole_consumer(sq);
        if (m2 < 0 || claimed_.count(m2) || !last_axis_mean(m2) || nodes_[m2].in[0] != sq) return false;
        const std::string var = nodes_[m2].out[0];
        const int ai = sole_consumer(var);
        if (!is_op(ai, "Add") || nodes_[ai].in.size() != 2 || nodes_[ai].out.size() != 1) return false;
        const Node& an = nodes_[ai];
        if ((an.in[0] == var) == (an.in[1] == var)) return false;
        float eps;
        if (!static_scalar(an.in[0] == var ? an.in[1] : an.in[0], &eps)) return false;
        const int qi = sole_consumer(an.out[0]);
        if (!is_op(qi, "Sqrt") || nodes_[qi].in.size() != 1 || nodes_[qi].out.size() != 1) return false;
        if (sole_consumer(nodes_[qi].out[0]) != di || nodes_[di].in[1] != nodes_[qi].out[0]) return false;
        mem = {si, pi, m2, ai, qi, di};
        std::string cur = nodes_[di].out[0], o;
        head.ln_scale.clear();
        head.ln_bias.clear();
        int k = sole_consumer(cur);
        if (is_op(k, "Mul") && affine_operand(k, cur, &o)) {
            head.ln_scale = o;
            mem.push_back(k);
            cur = nodes_[k].out[0];
            k = sole_consumer(cur);
        }
        if (is_op(k, "Add") && affine_operand(k, cur, &o)) {
            head.ln_bias = o;
            mem.push_back(k);
            cur = nodes_[k].out[0];
        }
        // a residual Add read only by the two nodes that read x
        head.ln_x = x;
        head.ln_res.clear();
        const int xi = producer(x);
        auto xc = gi_.consumers.find(x);
        if (is_op(xi, "Add") && nodes_[xi].in.size() == 2 && nodes_[xi].out.size() == 1 && !outs_.count(x) &&
            xc != gi_.consumers.end() && xc->second.size() == 2 && !static_f32(nodes_[xi].in[0]) &&
            !static_f32(nodes_[xi].in[1])) {
            head.ln_x = nodes_[xi].in[0];
            head.ln_res = nodes_[xi].in[1];
            mem.push_back(xi);
        }
        head.kind = Kind::FusedHead;
        head.pattern = Pattern::DecomposedLayerNorm;
        head.eps = eps;
        head.out = cur;
        return true;
    }

    // [B,S,H*D] --Reshape--> [B,S,H,D] --Transpose(perm)--> ; returns the Reshape input
    // t = Transpose(perm)(Reshape(src, shape)), or the same permutation as two Transposes in a
    // row (an export writes k.transpose(1, 2).transpose(2, 3)); the shape is a 4-element Int64
    // initializer or a tensor computed at run time (checked then).
    bool split_heads(const std::string& t, std::initializer_list<int64_t> perm, std::string* src,
                     std::string* shape, std::vector<int>& mem) const {
        const std::vector<int64_t> want(perm);
        const int ti = producer(t);
        if (!is_op(ti, "Transpose") || sole_consumer(t) < 0) return false;
        auto pa = nodes_[ti].iattrs.find("perm");
        if (pa == nodes_[ti].iattrs.end() || pa->second.size() != 4) return false;
        std::vector<int> m = {ti};
        std::string r_out = nodes_[ti].in[0];
        if (pa->second != want) {  // Transpose(p2)(Transpose(p1)(.)): out dim d = in dim p1[p2[d]]
            const int t1 = producer(r_out);
            if (!is_op(t1, "Transpose") || sole_consumer(r_out) != ti) return false;
            auto p1 = nodes_[t1].iattrs.find("perm");
            if (p1 == nodes_[t1].iattrs.end() || p1->second.size() != 4) return false;
            std::vector<int64_t> c(4);
            for (int d = 0; d < 4; ++d) {
                const int64_t j = pa->second[d];
                if (j < 0 || j > 3) return false;
                c[d] = p1->second[(size_t)j];
            }
            if (c != want) return false;
            m.push_back(t1);
            r_out = nodes_[t1].in[0];
        }
        const int ri = producer(r_out);
        if (!is_op(ri, "Reshape") || nodes_[ri].in.size() != 2 || sole_consumer(r_out) != m.back()) return false;
        auto sh = g_.inits.find(nodes_[ri].in[1]);
        if (sh != g_.inits.end() && (sh->second.dtype != ICX_I64 || numel(sh->second.shape) != 4)) return false;
        *src = nodes_[ri].in[0];
        *shape = nodes_[ri].in[1];
        mem.insert(mem.end(), m.begin(), m.end());
        mem.push_back(ri);
        return true;
    }
    // Every reader of t is one of `ok` (and t is not a live output).
    bool only_read_by(const std::string& t, std::initializer_list<int> ok) const {
        if (outs_.count(t)) return false;
        auto it = gi_.consumers.find(t);
        if (it == gi_.consumers.end()) return false;
        for (int c : it->second)
            if (std::find(ok.begin(), ok.end(), c) == ok.end()) return false;
        return true;
    }

    // DequantizeLinear(Gather(table, indices, axis 0), scale, [zp]) of an 8-bit table
    // initializer [V, D] with a per-tensor scale and zero point, the Gather read only by the
    // DequantizeLinear: an INT8 model's embedding lookup, one launch (the members run one by
    // one when the run-time shapes fall outside the kernel).
    bool match_gather_dequant(int di, PlannedOp& head, std::vector<int>& mem) {
        const Node& dq = nodes_[di];
        if (dq.op != "DequantizeLinear" || dq.in.size() < 2 || dq.in.size() > 3 || dq.out.size() != 1) return false;
        const int gi = producer(dq.in[0]);
        if (!is_op(gi, "Gather") || nodes_[gi].in.size() != 2 || sole_consumer(dq.in[0]) != di ||
            nodes_[gi].attr_or("axis", 0) != 0)
            return false;
        auto tb = g_.inits.find(nodes_[gi].in[0]);
        if (tb == g_.inits.end() || (tb->second.dtype != ICX_U8 && tb->second.dtype != ICX_I8) ||
            tb->second.shape.size() != 2)
            return false;
        auto sc = g_.inits.find(dq.in[1]);
        if (sc == g_.inits.end() || sc->second.dtype != ICX_F32 || numel(sc->second.shape) != 1) return false;
        if (dq.in.size() == 3 && !dq.in[2].empty()) {
            auto zp = g_.inits.find(dq.in[2]);
            if (zp == g_.inits.end() || zp->second.dtype != tb->second.dtype || numel(zp->second.shape) != 1)
                return false;
            head.w_zp = dq.in[2];
        }
        head.w = nodes_[gi].in[0];
        head.a = nodes_[gi].in[1];
        head.w_scale = dq.in[1];
        head.kind = Kind::FusedHead;
        head.pattern = Pattern::GatherDequantize;
        head.out = dq.out[0];
        mem = {gi};
        return true;
    }

    // Anchored at the Softmax of a BERT self-attention.
    bool match_attention(int si, PlannedOp& head, std::vector<int>& mem) {
        const Node& sm = nodes_[si];
        if (sm.op != "Softmax" || sm.in.size() != 1 || sm.out.size() != 1) return false;
        const int64_t axis = sm.attr_or("axis", -1);
        if (axis != -1 && axis != 3) return false;
        std::vector<int> m;
        std::string s = sm.in[0];
        int next = si;  // the member that reads s
        // padding mask: Where(cond, fill, scores) read only by the Softmax, fill a static scalar;
        // cond = Expand(mask, shape) — absorbed, with a Shape of the scores feeding it — or the
        // mask itself (checked at run time to broadcast as [B, 1, 1, S])
        int shape_reader = -1;
        const int wi = producer(s);
        if (is_op(wi, "Where") && nodes_[wi].in.size() == 3 && sole_consumer(s) == si &&
            static_scalar(nodes_[wi].in[1], &head.fill)) {
            std::string cond = nodes_[wi].in[0];
            const int ei = producer(cond);
            if (is_op(ei, "Expand") && nodes_[ei].in.size() == 2 && sole_consumer(cond) == wi) {
                const int shi = producer(nodes_[ei].in[1]);
                if (is_op(shi, "Shape") && nodes_[shi].in.size() == 1 && nodes_[shi].in[0] == nodes_[wi].in[2] &&
                    !nodes_[shi].attr.count("start") && !nodes_[shi].attr.count("end") &&
                    sole_consumer(nodes_[ei].in[1]) == ei) {
                    m.push_back(shi);
                    shape_reader = shi;
                } else {
                    head.mask_shape = nodes_[ei].in[1];  // must equal the scores' shape at run time
                }
                m.push_back(ei);
                cond = nodes_[ei].in[0];
            }
            head.mask = cond;
            m.push_back(wi);
            s = nodes_[wi].in[2];
            next = wi;
        }
        // scores scale: Div / Mul by a scalar, on the scores or on Q
        bool scaled = false;
        int pi = producer(s);
        if ((is_op(pi, "Div") || is_op(pi, "Mul")) && nodes_[pi].in.size() == 2 &&
            only_read_by(s, {next, shape_reader}) && static_scalar(nodes_[pi].in[1], &head.scale)) {
            head.scale_div = nodes_[pi].op == "Div";
            head.scale_q = false;
            scaled = true;
            m.push_back(pi);
            s = nodes_[pi].in[0];
            next = pi;
        }
        const int m1 = producer(s);
        if (!is_op(m1, "MatMul") || nodes_[m1].in.size() != 2 || !only_read_by(s, {next, shape_reader})) return false;
        m.push_back(m1);
        std::string qa = nodes_[m1].in[0];
        const int qs = producer(qa);
        if (!scaled && (is_op(qs, "Div") || is_op(qs, "Mul")) && nodes_[qs].in.size() == 2 &&
            sole_consumer(qa) == m1 && static_scalar(nodes_[qs].in[1], &head.scale)) {
            head.scale_div = nodes_[qs].op == "Div";
            head.scale_q = true;
            scaled = true;
            m.push_back(qs);
            qa = nodes_[qs].in[0];
        }
        if (!scaled) {
            head.scale = 1.0f;
            head.scale_div = false;
            head.scale_q = false;
        }
        if (!split_heads(qa, {0, 2, 1, 3}, &head.q, &head.q_shape, m)) return false;
        if (!split_heads(nodes_[m1].in[1], {0, 2, 3, 1}, &head.k, &head.k_shape, m)) return false;
        const int m2 = sole_consumer(sm.out[0]);
        if (!is_op(m2, "MatMul") || nodes_[m2].in.size() != 2 || nodes_[m2].in[0] != sm.out[0]) return false;
        m.push_back(m2);
        if (!split_heads(nodes_[m2].in[1], {0, 2, 1, 3}, &head.v, &head.v_shape, m)) return false;
        const int ot = sole_consumer(nodes_[m2].out[0]);
        if (!is_op(ot, "Transpose") || !has_perm(ot, {0, 2, 1, 3})) return false;
        const int orr = sole_consumer(nodes_[ot].out[0]);
        if (!is_op(orr, "Reshape") || nodes_[orr].in.size() != 2) return false;
        auto osh = g_.inits.find(nodes_[orr].in[1]);
        if (osh != g_.inits.end() && (osh->second.dtype != ICX_I64 || numel(osh->second.shape) != 3)) return false;
        m.push_back(ot);
        m.push_back(orr);
        auto qsh = g_.inits.find(head.q_shape);  // else the split is known at run time only
        if (qsh != g_.inits.end()) {
            const int64_t* d = reinterpret_cast<const int64_t*>(qsh->second.data.data());
            head.heads = d[2];
            head.head_dim = d[3];
        }
        head.o_shape = nodes_[orr].in[1];
        head.kind = Kind::FusedHead;
        head.pattern = Pattern::Attention;
        head.out = nodes_[orr].out[0];
        mem = m;
        return true;
    }
};

// ---------------------------------------------------------------------------------------
// run time
// ---------------------------------------------------------------------------------------

// How an operand of shape `o` broadcasts over an output of shape `x` (aligned at the right,
// numpy rules), in the kernels' terms; -1 when it would change x's shape or is none of
// scalar / [.., cols] / [.., rows, 1] / full.
int bcast_kind(const std::vector<int64_t>& o, const std::vector<int64_t>& x) {
    const size_t off = o.size() > x.size() ? o.size() - x.size() : 0;
    for (size_t i = 0; i < off; ++i)
        if (o[i] != 1) return -1;
    std::vector<int64_t> p(x.size(), 1);
    for (size_t i = off; i < o.size(); ++i) p[x.size() - (o.size() - i)] = o[i];
    for (size_t i = 0; i < x.size(); ++i)
        if (p[i] != 1 && p[i] != x[i]) return -1;
    if (numel(p) == 1) return ICX_BCAST_SCALAR;
    if (p == x) return ICX_BCAST_FULL;
    bool col = true;
    for (size_t i = 0; i + 1 < x.size(); ++i) col = col && p[i] == 1;
    if (col) return ICX_BCAST_COL;
    bool row = p.back() == 1;
    for (size_t i = 0; i + 1 < x.size(); ++i) row = row && p[i] == x[i];
    return row ? ICX_BCAST_ROW : -1;
}

std::vector<int64_t> broadcast_shape(const std::vector<int64_t>& a, const std::vector<int64_t>& b, bool* ok) {
    const size_t r = std::max(a.size(), b.size());
    std::vector<int64_t> s(r, 1);
    *ok = true;
    for (size_t i = 0; i < r; ++i) {
        const int64_t da = i < r - a.size() ? 1 : a[i - (r - a.size())];
        const int64_t db = i < r - b.size() ? 1 : b[i - (r - b.size())];
        if (da != db && da != 1 && db != 1) *ok = false;
        s[i] = da == 1 ? db : da;
    }
    return s;
}

// ONNX Reshape target (src/operators/reshape.rs): 0 copies the input dim (allowzero = 0),
// one -1 is inferred.
int reshape_target(const std::vector<int64_t>& in, const std::vector<int64_t>& spec, bool allowzero,
                   std::vector<int64_t>* out) {
    out->assign(spec.begin(), spec.end());
    int infer = -1;
    int64_t known = 1;
    for (size_t i = 0; i < spec.size(); ++i) {
        if (spec[i] == 0 && !allowzero) {
            if (i >= in.size()) {
                set_error("Reshape: 0 at axis %zu copies a dimension the input does not have", i);
                return ICX_ERR_SHAPE;
            }
            (*out)[i] = in[i];
        } else if (spec[i] == -1) {
            if (infer >= 0) {
                set_error("Reshape: more than one -1 in the target shape");
                return ICX_ERR_SHAPE;
            }
            infer = (int)i;
            continue;
        } else if (spec[i] < -1) {
            set_error("Reshape: invalid target dimension %lld", (long long)spec[i]);
            return ICX_ERR_SHAPE;
        }
        known *= (*out)[i];
    }
    const int64_t total = numel(in);
    if (infer >= 0) {
        if (known == 0 || total % known) {
            set_error("Reshape: cannot infer the -1 dimension of %s for %lld elements",
                      shape_str(spec).c_str(), (long long)total);
            return ICX_ERR_SHAPE;
        }
        (*out)[infer] = total / known;
    }
    if (numel(*out) != total) {
        set_error("Reshape: target %s has %lld elements, input %s has %lld", shape_str(*out).c_str(),
                  (long long)numel(*out), shape_str(in).c_str(), (long long)total);
        return ICX_ERR_SHAPE;
    }
    return ICX_OK;
}

// ---- tensors known on the host ------------------------------------------------------------
// An exported encoder computes its reshape targets, Slice bounds and Expand shapes from Shape
// results: small integer tensors.  The reference reads such Int64 tensors on the host and
// caches them (cache_i64 / get_or_fetch_i64, src/cuda/executor/layout.rs:136-146, 345-445),
// while each op of the shape arithmetic still runs as a GPU kernel.  Here an op whose inputs
// are all known on the host (computed on the host this run, a small initializer, or a small
// input bound from host memory) and whose output is small is computed on the host, and its
// output reaches device memory only if a device op or the caller reads it.
constexpr int64_t kHostFoldMax = 1024;  // elements

std::vector<int64_t> dense_strides(const std::vector<int64_t>& sh) {
    std::vector<int64_t> st(sh.size());
    int64_t s = 1;
    for (size_t i = sh.size(); i-- > 0;) {
        st[i] = s;
        s *= sh[i];
    }
    return st;
}

// Element strides with which a dense tensor of shape `in` is read over `out` (numpy rules,
// aligned at the right): 0 on a broadcast dimension.
std::vector<int64_t> bcast_strides(const std::vector<int64_t>& in, const std::vector<int64_t>& out) {
    std::vector<int64_t> st(out.size(), 0);
    const std::vector<int64_t> ds = dense_strides(in);
    const size_t off = out.size() - in.size();
    for (size_t i = 0; i < in.size(); ++i) st[off + i] = in[i] == 1 ? 0 : ds[i];
    return st;
}

// f(e, off) for every flat index e of `dims` in row-major order, off[k] = the element offset
// of operand k (base[k] + sum of index * st[k]).
template <typename F>
void for_each_offset(const std::vector<int64_t>& dims, const std::vector<std::vector<int64_t>>& st,
                     const std::vector<int64_t>& base, F f) {
    const int64_t total = numel(dims);
    const size_t r = dims.size();
    std::vector<int64_t> idx(r, 0), off = base;
    for (int64_t e = 0; e < total; ++e) {
        f(e, off);
        for (size_t d = r; d-- > 0;) {
            ++idx[d];
            for (size_t k = 0; k < st.size(); ++k) off[k] += st[k][d];
            if (idx[d] < dims[d]) break;
            for (size_t k = 0; k < st.size(); ++k) off[k] -= st[k][d] * dims[d];
            idx[d] = 0;
        }
    }
}

bool int_dtype(int dt) { return dt == ICX_I64 || dt == ICX_I32 || dt == ICX_I8 || dt == ICX_U8 || dt == ICX_BOOL; }

int64_t int_at(const HostTensor& t, int64_t i) {
    const uint8_t* p = t.data.data();
    switch (t.dtype) {
        case ICX_I64: return reinterpret_cast<const int64_t*>(p)[i];
        case ICX_I32: return reinterpret_cast<const int32_t*>(p)[i];
        case ICX_I8: return reinterpret_cast<const int8_t*>(p)[i];
        default: return p[i];  // UInt8, Bool
    }
}

void put_int(HostTensor& t, int64_t i, int64_t v) {
    uint8_t* p = t.data.data();
    switch (t.dtype) {
        case ICX_I64: reinterpret_cast<int64_t*>(p)[i] = v; break;
        case ICX_I32: reinterpret_cast<int32_t*>(p)[i] = (int32_t)v; break;
        case ICX_I8: reinterpret_cast<int8_t*>(p)[i] = (int8_t)v; break;
        case ICX_BOOL: p[i] = v != 0; break;
        default: p[i] = (uint8_t)v; break;
    }
}

HostTensor host_tensor(int dtype, const std::vector<int64_t>& shape) {
    HostTensor t;
    t.dtype = dtype;
    t.shape = shape;
    t.data.assign((size_t)numel(shape) * dtype_size(dtype), 0);
    return t;
}

// Slice parameters as the reference's GPU Slice normalises them (gpu_slice_nd,
// src/cuda/ops/layout/mod.rs:2849-2935; starts / ends of different lengths broadcast or
// truncate first, layout.rs:386-401; axes or steps of another length are ignored,
// layout.rs:403-445): per dimension the first index, the step and the output length.
int slice_params(const std::vector<int64_t>& shape, std::vector<int64_t> starts, std::vector<int64_t> ends,
                 const std::vector<int64_t>* axes_in, const std::vector<int64_t>* steps_in,
                 std::vector<int64_t>* first, std::vector<int64_t>* step, std::vector<int64_t>* len) {
    if (starts.size() != ends.size()) {
        if (starts.size() == 1 && ends.size() > 1) starts.assign(ends.size(), starts[0]);
        else if (ends.size() == 1 && starts.size() > 1) ends.assign(starts.size(), ends[0]);
        else {
            const size_t n = std::min(starts.size(), ends.size());
            starts.resize(n);
            ends.resize(n);
        }
    }
    const size_t ns = starts.size();
    std::vector<int64_t> axes, steps(ns, 1);
    if (axes_in && axes_in->size() == ns) axes = *axes_in;
    else for (size_t i = 0; i < ns; ++i) axes.push_back((int64_t)i);
    if (steps_in && steps_in->size() == ns) steps = *steps_in;
    const int64_t nd = (int64_t)shape.size();
    first->assign(nd, 0);
    step->assign(nd, 1);
    len->assign(shape.begin(), shape.end());
    std::vector<int64_t> end(shape.begin(), shape.end());
    for (size_t i = 0; i < ns; ++i) {
        const int64_t ax = axes[i] < 0 ? nd + axes[i] : axes[i];
        if (ax < 0 || ax >= nd) {
            set_error("Slice: axis %lld out of bounds for ndim %lld", (long long)axes[i], (long long)nd);
            return ICX_ERR_SHAPE;
        }
        if (steps[i] == 0) {
            set_error("Slice: step cannot be 0");
            return ICX_ERR_INVALID_ARG;
        }
        const int64_t dim = shape[ax];
        int64_t s = starts[i] < 0 ? std::max<int64_t>(dim + starts[i], 0) : std::min(starts[i], dim);
        int64_t e = ends[i] < 0 ? std::max<int64_t>(dim + ends[i], 0) : std::min(ends[i], dim);
        if (steps[i] < 0) {
            s = std::min(s, dim - 1);
            e = std::max<int64_t>(e, -1);
        } else {
            s = std::max<int64_t>(s, 0);
            e = std::max<int64_t>(e, 0);
        }
        (*first)[ax] = s;
        (*step)[ax] = steps[i];
        end[ax] = e;
    }
    for (int64_t d = 0; d < nd; ++d) {
        const int64_t s = (*first)[d], e = end[d], st = (*step)[d];
        // the reference's output length (layout/mod.rs:2931-2939)
        const int64_t n = st > 0 ? (e - s + st - 1) / st : (s - e - st - 1) / (-st);
        (*len)[d] = std::max<int64_t>(n, 0);
    }
    return ICX_OK;
}

class Runner {
   public:
    Runner(icx_graph& g, hipStream_t s) : g_(g), s_(s) {}

    int bind_inputs() {
        for (auto& kv : g_.bound) {
            const BoundInput& b = kv.second;
            if (b.dev) {
                DevTensor t;
                t.ptr = const_cast<void*>(b.dev);
                t.dtype = b.dtype;
                t.shape = b.shape;
                t.bytes = (size_t)numel(b.shape) * dtype_size(b.dtype);
                g_.values[kv.first] = t;
                continue;
            }
            DevTensor* d;
            int rc = alloc(kv.first, b.dtype, b.shape, &d);
            if (rc) return rc;
            if (d->bytes) ICX_HIP_CHECK(hipMemcpyAsync(d->ptr, b.host.data(), d->bytes, hipMemcpyHostToDevice, s_));
        }
        return ICX_OK;
    }

    int dispatch(const PlannedOp& op) {
        if (op.kind == Kind::FusedHead) {
            switch (op.pattern) {
                case Pattern::QuantizedLinear: return run_qlinear(op);
                case Pattern::Attention: return run_attention(op);
                case Pattern::AddLayerNorm:
                case Pattern::DecomposedLayerNorm:
                    return run_layer_norm(op.ln_x, op.ln_res, op.ln_scale, op.ln_bias, op.eps, op.out,
                                          pattern_name(op.pattern));
                case Pattern::GatherDequantize: return run_gather_dequant(op);
                default: return run_chain(op.chain_in, op.steps, op.out, pattern_name(op.pattern));
            }
        }
        return run_node(op.node);
    }

    // Return to the pool every pooled tensor whose last reader was plan entry i, or that
    // nothing reads.  Live outputs (and buffers they alias) stay until the next run.
    void release_dead(size_t i) {
        for (auto it = g_.values.begin(); it != g_.values.end();) {
            const std::string& name = it->first;
            std::string key = name;
            size_t sfx = name.rfind("::rowsum");
            if (sfx == std::string::npos) sfx = name.rfind("::range");
            if (sfx != std::string::npos) key = name.substr(0, sfx);
            auto lu = g_.last_use.find(key);
            const bool dead = !g_.keep.count(name) && (lu == g_.last_use.end() || lu->second <= i);
            if (dead) {
                if (it->second.pooled) g_.pool.put(it->second.ptr, it->second.cls);
                it = g_.values.erase(it);
            } else {
                ++it;
            }
        }
    }

   private:
    icx_graph& g_;
    hipStream_t s_;

    int run_node(const Node& n) {
        const std::string& t = n.op;
        if (t == "DynamicQuantizeLinear") return run_dql(n);
        if (t == "MatMulInteger") return run_matmul_integer(n);
        if (t == "DequantizeLinear") return run_dequantize(n);
        if (t == "Cast") return run_cast(n);
        if (t == "LayerNormalization") {
            const DevTensor* x = n.in.empty() ? nullptr : find(n.in[0]);
            const int64_t axis = n.attr_or("axis", -1);
            if (n.in.size() != 3 || !x || (axis != -1 && axis != (int64_t)x->shape.size() - 1)) {
                set_error("LayerNormalization: only the last axis, with scale and bias, is on this path");
                return ICX_ERR_UNSUPPORTED;
            }
            return run_layer_norm(n.in[0], "", n.in[1], n.in[2], (float)n.fattr_or("epsilon", 1e-5), n.out[0],
                                  "LayerNormalization");
        }
        if (t == "Softmax") return run_softmax(n);
        if (t == "Erf") {
            Step st;
            st.op = ICX_OP_ERF;
            return run_chain(n.in[0], {st}, n.out[0], "Erf");
        }
        if (t == "Transpose") return run_transpose(n);
        if (t == "Reshape") return run_reshape(n);
        if (t == "MatMul") return run_matmul_f32(n);
        if (t == "Gather") return run_gather(n);
        if (t == "ReduceMean") return run_reduce_mean(n);
        if (t == "Pow") return run_pow(n);
        if (t == "Sqrt") return run_sqrt(n);
        if (t == "Shape") return run_shape(n);
        if (t == "Unsqueeze" || t == "Squeeze" || t == "Identity") return run_view(n);
        if (t == "Concat") return run_concat(n);
        if (t == "Slice") return run_slice(n);
        if (t == "Expand") return run_expand(n);
        if (t == "Equal") return run_equal(n);
        if (t == "Where") return run_where(n);
        if (op_code(t) >= 0) return run_binary(n);
        set_error("op '%s' is not on the quantized-linear path", t.c_str());
        return ICX_ERR_UNSUPPORTED;
    }

    const DevTensor* find(const std::string& name) const {
        auto v = g_.values.find(name);
        if (v != g_.values.end()) return &v->second;
        auto w = g_.weights.find(name);
        if (w != g_.weights.end()) return &w->second;
        return nullptr;
    }
    int need(const std::string& name, const DevTensor** out, const char* who) const {
        *out = find(name);
        if (*out) return ICX_OK;
        if (g_.hv.count(name)) return materialize(name, out);
        set_error("%s: input tensor '%s' is missing", who, name.c_str());
        return ICX_ERR_INVALID_ARG;
    }
    // A tensor computed on the host, uploaded for a device reader (through kernel arguments,
    // so a captured run replays the copy); it stays a host value too.
    int materialize(const std::string& name, const DevTensor** out) const {
        const HostTensor& h = g_.hv.at(name);
        DevTensor t;
        t.dtype = h.dtype;
        t.shape = h.shape;
        t.bytes = h.data.size();
        t.ptr = g_.pool.get(std::max<size_t>(t.bytes, 1), &t.cls);
        if (!t.ptr) {
            set_error("memory pool: hipMalloc of %zu bytes for '%s' failed", t.bytes, name.c_str());
            return ICX_ERR_HIP;
        }
        t.pooled = true;
        DevTensor& d = g_.values[name] = t;
        *out = &d;
        return icx::upload_bytes(s_, h.data.data(), h.data.size(), d.ptr);
    }
    // The host copy of `name` if it is known on the host without reading device memory.
    const HostTensor* host_known(const std::string& name) const {
        auto h = g_.hv.find(name);
        if (h != g_.hv.end()) return &h->second;
        auto it = g_.inits.find(name);
        if (it != g_.inits.end()) return numel(it->second.shape) <= kHostFoldMax ? &it->second : nullptr;
        auto b = g_.bound.find(name);
        if (b != g_.bound.end() && !b->second.dev && numel(b->second.shape) <= kHostFoldMax) {
            HostTensor t;
            t.dtype = b->second.dtype;
            t.shape = b->second.shape;
            t.data = b->second.host;
            return &(g_.hv[name] = std::move(t));
        }
        return nullptr;
    }
    // Integer values of `name` on the host (Float32 truncated, as the reference's Slice and
    // ReduceMean read their parameters): a host-known tensor, else read from the device
    // (synchronising the stream, as the reference's get_or_fetch_i64 does; refused while
    // the stream is being captured) and kept for later readers.
    int host_ints(const std::string& name, std::vector<int64_t>* v, const char* who) const {
        const HostTensor* h = host_known(name);
        if (!h) {
            const DevTensor* d = find(name);
            if (!d) {
                set_error("%s: input tensor '%s' is missing", who, name.c_str());
                return ICX_ERR_INVALID_ARG;
            }
            if (!int_dtype(d->dtype) && d->dtype != ICX_F32) {
                set_error("%s: '%s' must be an integer tensor, got %s", who, name.c_str(), dtype_name(d->dtype));
                return ICX_ERR_DTYPE;
            }
            if (numel(d->shape) > kHostFoldMax) {
                set_error("%s: '%s' has %lld elements, too many to read on the host", who, name.c_str(),
                          (long long)numel(d->shape));
                return ICX_ERR_SHAPE;
            }
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            ICX_HIP_CHECK(hipStreamIsCapturing(s_, &cs));
            if (cs != hipStreamCaptureStatusNone) {
                set_error("%s: '%s' would have to be read on the host while the run is captured", who, name.c_str());
                return ICX_ERR_UNSUPPORTED;
            }
            HostTensor t;
            t.dtype = d->dtype;
            t.shape = d->shape;
            t.data.resize(d->bytes);
            if (d->bytes) {
                ICX_HIP_CHECK(hipMemcpyAsync(t.data.data(), d->ptr, d->bytes, hipMemcpyDeviceToHost, s_));
                ICX_HIP_CHECK(hipStreamSynchronize(s_));
            }
            h = &(g_.hv[name] = std::move(t));
        }
        v->resize((size_t)numel(h->shape));
        for (size_t i = 0; i < v->size(); ++i)  // (Float32 as the reference's Slice / ReduceMean take it)
            (*v)[i] = h->dtype == ICX_F32 ? (int64_t)reinterpret_cast<const float*>(h->data.data())[i]
                                          : int_at(*h, (int64_t)i);
        return ICX_OK;
    }
    // Shape and dtype of a tensor wherever it lives (no upload).
    bool shape_of(const std::string& name, std::vector<int64_t>* sh, int* dt) const {
        if (const DevTensor* d = find(name)) {
            *sh = d->shape;
            *dt = d->dtype;
            return true;
        }
        auto h = g_.hv.find(name);
        if (h == g_.hv.end()) return false;
        *sh = h->second.shape;
        *dt = h->second.dtype;
        return true;
    }
    // Every non-empty input of the first n_inputs an integer or Bool tensor known on the
    // host: the op is shape arithmetic and is computed on the host (Float32 tensors, the
    // model's activations and constants, always take the device kernels).
    bool all_host(const Node& n, size_t n_inputs, std::vector<const HostTensor*>* hs) const {
        hs->assign(n_inputs, nullptr);
        for (size_t i = 0; i < n_inputs && i < n.in.size(); ++i) {
            if (n.in[i].empty()) continue;
            (*hs)[i] = host_known(n.in[i]);
            if (!(*hs)[i] || !int_dtype((*hs)[i]->dtype)) return false;
        }
        return true;
    }
    // (a host route returns kHostTooLarge, having done nothing, for an output of more than
    // kHostFoldMax elements: the op then runs on the device)
    static constexpr int kHostTooLarge = -1;
    int set_host(const std::string& name, HostTensor t) const {
        g_.hv[name] = std::move(t);
        return ICX_OK;
    }
    int alloc(const std::string& name, int dtype, const std::vector<int64_t>& shape, DevTensor** out) {
        auto old = g_.values.find(name);
        if (old != g_.values.end()) {
            if (old->second.pooled) g_.pool.put(old->second.ptr, old->second.cls);
            g_.values.erase(old);
        }
        DevTensor t;
        t.dtype = dtype;
        t.shape = shape;
        t.bytes = (size_t)numel(shape) * dtype_size(dtype);
        t.ptr = g_.pool.get(std::max<size_t>(t.bytes, 1), &t.cls);
        if (!t.ptr) {
            set_error("memory pool: hipMalloc of %zu bytes for '%s' failed", t.bytes, name.c_str());
            return ICX_ERR_HIP;
        }
        t.pooled = true;
        *out = &(g_.values[name] = t);
        return ICX_OK;
    }
    // Partials buffer of `out` when a DynamicQuantizeLinear reads it (null otherwise).
    int range_parts(const std::string& out, float2** part) {
        *part = nullptr;
        if (!g_.range_wanted.count(out)) return ICX_OK;
        DevTensor* P;
        int rc = alloc(out + "::range", ICX_F32, {2 * (int64_t)icx::kMaxRangeParts}, &P);
        if (rc) return rc;
        *part = static_cast<float2*>(P->ptr);
        return ICX_OK;
    }
    void record_range(const std::string& out, int n_part) {
        if (n_part > 0) g_.range_of[out] = {out + "::range", n_part};
    }

    int workspace(size_t bytes) {
        if (bytes <= g_.ws_bytes) return ICX_OK;
        if (g_.ws) {
            ICX_HIP_CHECK(hipStreamSynchronize(s_));  // earlier ops on the stream may read it
            ICX_HIP_CHECK(hipFree(g_.ws));
            g_.ws = nullptr;
            g_.ws_bytes = 0;
        }
        ICX_HIP_CHECK(hipMalloc(&g_.ws, bytes));
        g_.ws_bytes = bytes;
        return ICX_OK;
    }
    int need_f32(const std::string& name, const DevTensor** out, const char* who) const {
        int rc = need(name, out, who);
        if (rc) return rc;
        if ((*out)->dtype == ICX_F32) return ICX_OK;
        set_error("%s: '%s' must be Float32, got %s", who, name.c_str(), dtype_name((*out)->dtype));
        return ICX_ERR_DTYPE;
    }

    int chain_operand(const std::string& name, const std::vector<int64_t>& out_shape, const char* who,
                      int32_t* kind, const float** p) const {
        const DevTensor* t;
        int rc = need_f32(name, &t, who);
        if (rc) return rc;
        *kind = bcast_kind(t->shape, out_shape);
        *p = static_cast<const float*>(t->ptr);
        if (*kind >= 0) return ICX_OK;
        set_error("%s: operand '%s' %s does not broadcast over %s", who, name.c_str(), shape_str(t->shape).c_str(),
                  shape_str(out_shape).c_str());
        return ICX_ERR_SHAPE;
    }
    int make_chain(const std::vector<Step>& steps, const std::vector<int64_t>& out_shape, icx_chain& ch,
                   const char* who) const {
        std::memset(&ch, 0, sizeof(ch));
        ch.n_ops = (int32_t)steps.size();
        for (size_t k = 0; k < steps.size(); ++k) {
            icx_chain_op& o = ch.ops[k];
            o.op = steps[k].op;
            o.operand_is_lhs = steps[k].lhs ? 1 : 0;
            if (steps[k].op > ICX_OP_DIV) continue;  // operand-free step
            int rc = chain_operand(steps[k].opnd0, out_shape, who, &o.kind0, &o.p0);
            if (rc) return rc;
            if (!steps[k].opnd1.empty()) {
                rc = chain_operand(steps[k].opnd1, out_shape, who, &o.kind1, &o.p1);
                if (rc) return rc;
            }
        }
        return ICX_OK;
    }

    // Zero point of a MatMulInteger operand: scalar (either side) or [N] (weight side).
    int zero_point(const std::string& name, int operand_dtype, bool weight_side, int64_t N, const void** ptr,
                   size_t* len) const {
        *ptr = nullptr;
        *len = 1;
        if (name.empty()) return ICX_OK;
        const DevTensor* z;
        int rc = need(name, &z, "MatMulInteger");
        if (rc) return rc;
        const char* which = weight_side ? "b_zero_point" : "a_zero_point";
        if (z->dtype != operand_dtype) {
            set_error("MatMulInteger: %s dtype %s must match its operand's dtype %s", which, dtype_name(z->dtype),
                      dtype_name(operand_dtype));
            return ICX_ERR_DTYPE;
        }
        const int64_t n = numel(z->shape);
        if (n == 1) {
            *len = 1;
        } else if (weight_side && z->shape.size() == 1 && n == N) {
            *len = (size_t)N;
        } else {
            set_error("MatMulInteger: %s of shape %s is not supported (scalar%s)", which, shape_str(z->shape).c_str(),
                      weight_side ? " or [N]" : "");
            return ICX_ERR_SHAPE;
        }
        *ptr = z->ptr;
        return ICX_OK;
    }

    // A [M,K] or [B,S,K] (flattened to [B*S, K], src/cuda/executor/layout.rs:1058-1090).
    int gemm_rows(const DevTensor* A, int64_t Kb, int64_t* M, std::vector<int64_t>* lead) const {
        if (A->dtype != ICX_U8 && A->dtype != ICX_I8) {
            set_error("MatMulInteger: a dtype %s unsupported (must be Int8 or UInt8)", dtype_name(A->dtype));
            return ICX_ERR_DTYPE;
        }
        if (A->shape.size() != 2 && A->shape.size() != 3) {
            set_error("MatMulInteger: a of rank %zu unsupported (2-D or 3-D x 2-D)", A->shape.size());
            return ICX_ERR_SHAPE;
        }
        if (A->shape.back() != Kb) {
            set_error("MatMulInteger: inner dims differ: a %s, b has K = %lld", shape_str(A->shape).c_str(),
                      (long long)Kb);
            return ICX_ERR_SHAPE;
        }
        lead->assign(A->shape.begin(), A->shape.end() - 1);
        *M = numel(*lead);
        return ICX_OK;
    }

    // A sibling group: one launch writes every member's output (segment s = member s).
    int run_qlinear_group(const PlannedOp& op) {
        const DevTensor* A;
        int rc = need(op.a, &A, "QuantizedLinear");
        if (rc) return rc;
        auto pk = g_.packed.find(op.group_w);
        if (pk == g_.packed.end()) {
            set_error("QuantizedLinear: group weight of '%s' was not packed at compile", op.node.name.c_str());
            return ICX_ERR_INVALID_ARG;
        }
        const PackedW& pw = pk->second;
        const int n_seg = (int)op.group_members.size();
        int64_t M;
        std::vector<int64_t> lead;
        rc = gemm_rows(A, pw.K, &M, &lead);
        if (rc) return rc;
        const void *azp, *bzp = nullptr;
        size_t alen;
        rc = zero_point(op.a_zp, A->dtype, false, pw.N, &azp, &alen);
        if (rc) return rc;
        const int32_t* rowsum = nullptr;
        auto rs = g_.rowsum_of.find(op.a);
        if (rs != g_.rowsum_of.end()) {
            const DevTensor* r = find(rs->second);
            if (r) rowsum = static_cast<const int32_t*>(r->ptr);
        }
        std::vector<int64_t> full = lead, part = lead;
        full.push_back(pw.N);
        part.push_back(pw.N / n_seg);
        icx_chain ch;
        rc = make_chain(op.group_steps, full, ch, "QuantizedLinear");
        if (rc) return rc;
        const void* a_ptr = A->ptr;
        const int a_dt = A->dtype;
        float* ys[icx::kMaxSegments] = {};
        for (int i = 0; i < n_seg; ++i) {
            DevTensor* Y;
            rc = alloc(g_.plan[op.group_members[i]].out, ICX_F32, part, &Y);
            if (rc) return rc;
            ys[i] = static_cast<float*>(Y->ptr);
        }
        rc = workspace(icx_matmul_integer_workspace_size(M, pw.K, pw.N, 1));
        if (rc) return rc;
        return icx::qlinear_f32_seg(s_, a_ptr, a_dt, pw.packed, pw.dtype, pw.colsum, M, pw.K, pw.N, azp, bzp, 1,
                                    rowsum, &ch, ys, n_seg, g_.ws, g_.ws_bytes);
    }

    // The head whose input's DQL it runs in the same launch: ICX_OK when that launch ran
    // (*done), else the DQL has run on its own and the head continues as usual.
    int run_qin(const PlannedOp& op, const Node& d, bool* done) {
        *done = false;
        const DevTensor* X;
        int rc = need_f32(d.in[0], &X, "DynamicQuantizeLinear");
        if (rc) return rc;
        auto pk = g_.packed.find(op.w);
        const int64_t K = X->shape.empty() ? 0 : X->shape.back();
        if (g_.qsync && pk != g_.packed.end() && K == pk->second.K && K > 0 && !X->shape.empty()) {
            const PackedW& pw = pk->second;
            const std::vector<int64_t> xshape = X->shape;
            const int64_t M = numel(xshape) / K;
            std::vector<int64_t> oshape(xshape.begin(), xshape.end() - 1);
            oshape.push_back(pw.N);
            DevTensor *QY, *QS, *QZ, *Y;
            rc = alloc(d.out[0], ICX_U8, xshape, &QY);
            if (!rc) rc = alloc(d.out[1], ICX_F32, {}, &QS);
            if (!rc) rc = alloc(d.out[2], ICX_U8, {}, &QZ);
            if (rc) return rc;
            icx_chain ch;
            rc = make_chain(op.steps, oshape, ch, "QuantizedLinear");
            if (!rc) rc = alloc(op.out, ICX_F32, oshape, &Y);
            if (rc) return rc;
            const float* x = static_cast<const float*>(find(d.in[0])->ptr);
            rc = icx::dql_qlinear(s_, x, (size_t)M, (size_t)K, static_cast<uint8_t*>(QY->ptr),
                                  static_cast<float*>(QS->ptr), static_cast<uint8_t*>(QZ->ptr), pw.packed, pw.dtype,
                                  pw.colsum, pw.N, &ch, static_cast<float*>(Y->ptr), g_.qsync);
            if (rc == ICX_OK) {
                ++g_.qin_fused;
                *done = true;
                return ICX_OK;
            }
            if (rc != ICX_ERR_UNSUPPORTED) return rc;
            icx::clear_error();  // shape outside the fused kernel: the DQL on its own, then the GEMM
        }
        return run_dql(d, true);
    }

    int run_qlinear(const PlannedOp& op) {
        if (!op.group.empty())  // members other than the lead were written by its launch
            return op.group_members.empty() ? ICX_OK : run_qlinear_group(op);
        auto qi = g_.qin.find(op.out);
        if (qi != g_.qin.end()) {
            bool done;
            int rc = run_qin(op, qi->second, &done);
            if (rc || done) return rc;
        }
        const DevTensor* A;
        int rc = need(op.a, &A, "QuantizedLinear");
        if (rc) return rc;
        auto pk = g_.packed.find(op.w);
        if (pk == g_.packed.end()) {
            set_error("QuantizedLinear: weight '%s' was not packed at compile", op.w.c_str());
            return ICX_ERR_INVALID_ARG;
        }
        const PackedW& pw = pk->second;
        int64_t M;
        std::vector<int64_t> oshape;
        rc = gemm_rows(A, pw.K, &M, &oshape);
        if (rc) return rc;
        oshape.push_back(pw.N);
        const void *azp, *bzp = nullptr;
        size_t alen, blen = 1;
        rc = zero_point(op.a_zp, A->dtype, false, pw.N, &azp, &alen);
        if (rc) return rc;
        if (!op.w_zp_folded) {
            rc = zero_point(op.w_zp, pw.dtype, true, pw.N, &bzp, &blen);
            if (rc) return rc;
        }
        const int32_t* rowsum = nullptr;
        auto rs = g_.rowsum_of.find(op.a);
        if (rs != g_.rowsum_of.end()) {
            const DevTensor* r = find(rs->second);
            if (r) rowsum = static_cast<const int32_t*>(r->ptr);
        }
        icx_chain ch;
        rc = make_chain(op.steps, oshape, ch, "QuantizedLinear");
        if (rc) return rc;
        const void* a_ptr = A->ptr;
        const int a_dt = A->dtype;
        auto qo = g_.quant_out.find(op.out);
        if (qo != g_.quant_out.end() && g_.qsync && bzp == nullptr) {
            const Node& d = qo->second;
            DevTensor *QY, *QS, *QZ;
            rc = alloc(d.out[0], ICX_U8, oshape, &QY);
            if (!rc) rc = alloc(d.out[1], ICX_F32, {}, &QS);
            if (!rc) rc = alloc(d.out[2], ICX_U8, {}, &QZ);
            if (rc) return rc;
            rc = icx::qlinear_dql(s_, a_ptr, a_dt, pw.packed, pw.dtype, pw.colsum, M, pw.K, pw.N, azp, &ch,
                                  static_cast<uint8_t*>(QY->ptr), static_cast<float*>(QS->ptr),
                                  static_cast<uint8_t*>(QZ->ptr), g_.qsync);
            if (rc == ICX_OK) {
                g_.dql_done.insert(d.out[0]);
                ++g_.quant_fused;
                return ICX_OK;
            }
            if (rc != ICX_ERR_UNSUPPORTED) return rc;
            icx::clear_error();  // shape outside the fused kernel: f32 output, then the DQL
        }
        DevTensor* Y;
        rc = alloc(op.out, ICX_F32, oshape, &Y);
        if (rc) return rc;
        rc = workspace(icx_matmul_integer_workspace_size(M, pw.K, pw.N, 1));
        if (rc) return rc;
        float2* part;
        rc = range_parts(op.out, &part);
        if (rc) return rc;
        int n_part = 0;
        rc = icx::qlinear_f32(s_, a_ptr, a_dt, pw.packed, pw.dtype, 1, pw.colsum, M, pw.K, pw.N, azp, bzp, blen,
                              rowsum, &ch, static_cast<float*>(Y->ptr), g_.ws, g_.ws_bytes, part, &n_part);
        if (!rc) record_range(op.out, n_part);
        return rc;
    }

    // Gather + DequantizeLinear of an 8-bit table in one launch, or the two nodes.
    int run_gather_dequant(const PlannedOp& op) {
        const DevTensor *T, *I, *S, *Z = nullptr;
        int rc = need(op.w, &T, "GatherDequantize");
        if (!rc) rc = need(op.a, &I, "GatherDequantize");
        if (!rc) rc = need(op.w_scale, &S, "GatherDequantize");
        if (!rc && !op.w_zp.empty()) rc = need(op.w_zp, &Z, "GatherDequantize");
        if (rc) return rc;
        if ((I->dtype == ICX_I64 || I->dtype == ICX_I32) && T->shape.size() == 2 && T->shape[1] % 4 == 0) {
            std::vector<int64_t> oshape = I->shape;
            oshape.push_back(T->shape[1]);
            const void *tb = T->ptr, *ix = I->ptr, *zp = Z ? Z->ptr : nullptr;
            const float* sc = static_cast<const float*>(S->ptr);
            const int tdt = T->dtype, idt = I->dtype;
            const size_t V = (size_t)T->shape[0], D = (size_t)T->shape[1], n = (size_t)numel(I->shape);
            DevTensor* Y;
            rc = alloc(op.out, ICX_F32, oshape, &Y);
            if (rc) return rc;
            rc = icx::gather_dequant_f32(s_, tb, tdt, V, D, ix, idt, n, sc, zp, static_cast<float*>(Y->ptr));
            if (rc != ICX_ERR_UNSUPPORTED) return rc;
            icx::clear_error();
        }
        for (const Node& m : op.sub) {
            rc = run_node(m);
            if (rc) return rc;
        }
        return ICX_OK;
    }

    // Fused attention, or its member nodes when the shapes are outside the kernel.
    int run_attention(const PlannedOp& op) {
        const DevTensor *Q, *K, *V;
        int rc = need_f32(op.q, &Q, "Attention");
        if (!rc) rc = need_f32(op.k, &K, "Attention");
        if (!rc) rc = need_f32(op.v, &V, "Attention");
        if (rc) return rc;
        int64_t heads = op.heads, head_dim = op.head_dim;
        bool fused = Q->shape.size() == 3 && Q->shape == K->shape && Q->shape == V->shape;
        if (fused && heads == 0) {  // reshape targets computed at run time: the split is Q's
            std::vector<int64_t> spec, tgt;
            fused = !host_ints(op.q_shape, &spec, "Attention") && !reshape_target(Q->shape, spec, false, &tgt) &&
                    tgt.size() == 4;
            if (fused) {
                heads = tgt[2];
                head_dim = tgt[3];
            }
        }
        fused = fused && head_dim == 64 && heads > 0 && Q->shape[2] == heads * head_dim && Q->shape[1] > 0 &&
                Q->shape[1] <= icx::kAttentionMaxSeq;
        std::vector<int64_t> split = {Q->shape.empty() ? 0 : Q->shape[0], Q->shape.size() > 1 ? Q->shape[1] : 0,
                                      heads, head_dim};
        for (const std::string* sh : {&op.q_shape, &op.k_shape, &op.v_shape}) {
            std::vector<int64_t> spec, tgt;
            if (!fused) break;
            if (host_ints(*sh, &spec, "Attention") || reshape_target(Q->shape, spec, false, &tgt) || tgt != split)
                fused = false;
        }
        std::vector<int64_t> oshape;
        if (fused) {
            std::vector<int64_t> spec;
            std::vector<int64_t> full = {Q->shape[0], Q->shape[1], heads, head_dim};
            if (host_ints(op.o_shape, &spec, "Attention") || reshape_target(full, spec, false, &oshape) ||
                oshape != Q->shape)
                fused = false;
        }
        // the padding mask: one byte per key, [B | 1, 1, 1, S] (right-aligned), every batch row
        // or one for all; an absorbed Expand must target the scores' shape
        icx::AttnMask mask;
        if (fused && !op.mask.empty()) {
            std::vector<int64_t> ms;
            int mdt;
            const int64_t B = Q->shape[0], S = Q->shape[1];
            fused = shape_of(op.mask, &ms, &mdt) && (mdt == ICX_BOOL || mdt == ICX_U8) && ms.size() <= 4 &&
                    !ms.empty() && ms.back() == S;
            while (fused && ms.size() < 4) ms.insert(ms.begin(), 1);
            fused = fused && ms[1] == 1 && ms[2] == 1 && (ms[0] == 1 || ms[0] == B);
            if (fused && !op.mask_shape.empty()) {
                std::vector<int64_t> tgt;
                fused = !host_ints(op.mask_shape, &tgt, "Attention") &&
                        tgt == std::vector<int64_t>{B, heads, S, S};
            }
            const DevTensor* M = nullptr;
            if (fused) {
                rc = need(op.mask, &M, "Attention");
                if (rc) return rc;
                mask.keys = static_cast<const uint8_t*>(M->ptr);
                mask.batch_stride = ms[0] == B && B > 1 ? S : 0;
                mask.fill = op.fill;
            }
        }
        icx::clear_error();
        if (!fused) {  // run the decomposed subgraph as the reference does
            for (const Node& m : op.sub) {
                rc = run_node(m);
                if (rc) return rc;
            }
            return ICX_OK;
        }
        const std::vector<int64_t> shape = Q->shape;
        const float *q = static_cast<const float*>(Q->ptr), *k = static_cast<const float*>(K->ptr),
                    *v = static_cast<const float*>(V->ptr);
        const size_t hd = (size_t)shape[2];
        auto qo = g_.quant_out.find(op.out);
        if (qo != g_.quant_out.end() && g_.qsync) {  // the context's only reader is a DQL
            const Node& d = qo->second;
            DevTensor *QY, *QS, *QZ;
            rc = alloc(d.out[0], ICX_U8, shape, &QY);
            if (!rc) rc = alloc(d.out[1], ICX_F32, {}, &QS);
            if (!rc) rc = alloc(d.out[2], ICX_U8, {}, &QZ);
            if (rc) return rc;
            rc = icx::attention_dql(s_, q, k, v, shape[0], shape[1], heads, head_dim, hd, hd, hd, hd, op.scale,
                                    op.scale_div ? 1 : 0, op.scale_q ? 1 : 0, mask.keys ? &mask : nullptr,
                                    static_cast<uint8_t*>(QY->ptr),
                                    static_cast<float*>(QS->ptr), static_cast<uint8_t*>(QZ->ptr), g_.qsync);
            if (rc == ICX_OK) {
                g_.dql_done.insert(d.out[0]);
                ++g_.quant_fused;
                return ICX_OK;
            }
            if (rc != ICX_ERR_UNSUPPORTED) return rc;
            icx::clear_error();  // a grid that would not be resident at once: f32 context, then the DQL
        }
        DevTensor* O;
        rc = alloc(op.out, ICX_F32, shape, &O);
        if (rc) return rc;
        float2* part;
        rc = range_parts(op.out, &part);
        if (rc) return rc;
        int n_part = 0;
        rc = icx::attention_f32(s_, q, k, v, shape[0], shape[1], heads, head_dim, hd, hd, hd, hd, op.scale,
                                op.scale_div ? 1 : 0, op.scale_q ? 1 : 0, mask.keys ? &mask : nullptr,
                                static_cast<float*>(O->ptr), part, &n_part);
        if (!rc) record_range(op.out, n_part);
        return rc;
    }

    int run_layer_norm(const std::string& xn, const std::string& resn, const std::string& sn, const std::string& bn,
                       float eps, const std::string& out, const char* who) {
        const DevTensor *X, *R = nullptr, *S = nullptr, *B = nullptr;  // no scale / bias: x 1, + (-0)
        int rc = need_f32(xn, &X, who);
        if (!rc && !resn.empty()) rc = need_f32(resn, &R, who);
        if (!rc && !sn.empty()) rc = need_f32(sn, &S, who);
        if (!rc && !bn.empty()) rc = need_f32(bn, &B, who);
        if (rc) return rc;
        size_t res_rows = 0;
        if (R && R->shape != X->shape) {
            // a residual of X's trailing shape (leading unit dims aside: position embeddings
            // [1, S, D] over [B, S, D]) is read row-periodically by the kernel; any other
            // broadcast is materialised first
            std::vector<int64_t> rs = R->shape;
            while (!rs.empty() && rs.front() == 1 && rs.size() > 1) rs.erase(rs.begin());
            bool periodic = !X->shape.empty() && rs.size() <= X->shape.size() && !rs.empty() &&
                            std::equal(rs.begin(), rs.end(), X->shape.end() - (ptrdiff_t)rs.size()) &&
                            numel(rs) > 0;
            if (periodic) {
                res_rows = (size_t)(numel(rs) / X->shape.back());
            } else {
                const std::string tmp = out + "::sum";
                rc = binary_f32_into(ICX_OP_ADD, xn, resn, tmp, who);
                if (rc) return rc;
                return run_layer_norm(tmp, "", sn, bn, eps, out, who);
            }
        }
        if (X->shape.empty()) {
            set_error("%s: input must have at least one axis", who);
            return ICX_ERR_SHAPE;
        }
        const int64_t cols = X->shape.back();
        if ((S && numel(S->shape) != cols) || (B && numel(B->shape) != cols)) {
            set_error("%s: scale %s / bias %s do not match the normalised axis (%lld)", who,
                      S ? shape_str(S->shape).c_str() : "-", B ? shape_str(B->shape).c_str() : "-", (long long)cols);
            return ICX_ERR_SHAPE;
        }
        const std::vector<int64_t> shape = X->shape;
        const float *x = static_cast<const float*>(X->ptr), *r = R ? static_cast<const float*>(R->ptr) : nullptr,
                    *sc = S ? static_cast<const float*>(S->ptr) : nullptr,
                    *bi = B ? static_cast<const float*>(B->ptr) : nullptr;
        DevTensor* Y;
        rc = alloc(out, ICX_F32, shape, &Y);
        if (rc) return rc;
        float2* part;
        rc = range_parts(out, &part);
        if (rc) return rc;
        int n_part = 0;
        rc = icx::layer_norm_f32(s_, x, r, res_rows, cols ? numel(shape) / cols : 0, cols, sc, bi, eps,
                                 static_cast<float*>(Y->ptr), part, &n_part);
        if (!rc) record_range(out, n_part);
        return rc;
    }

    int run_softmax(const Node& n) {
        const DevTensor* X;
        int rc = need_f32(n.in[0], &X, "Softmax");
        if (rc) return rc;
        const int64_t rank = (int64_t)X->shape.size();
        const int64_t axis = n.attr_or("axis", -1);
        if (rank == 0 || (axis != -1 && axis != rank - 1)) {
            set_error("Softmax: only the last axis is on this path (axis %lld of rank %lld)", (long long)axis,
                      (long long)rank);
            return ICX_ERR_UNSUPPORTED;
        }
        const std::vector<int64_t> shape = X->shape;
        const float* x = static_cast<const float*>(X->ptr);
        DevTensor* Y;
        rc = alloc(n.out[0], ICX_F32, shape, &Y);
        if (rc) return rc;
        const int64_t cols = shape.back();
        return icx_softmax_f32(s_, x, cols ? numel(shape) / cols : 0, cols, static_cast<float*>(Y->ptr));
    }

    int run_transpose(const Node& n) {
        const DevTensor* X;
        int rc = need(n.in[0], &X, "Transpose");
        if (rc) return rc;
        const int rank = (int)X->shape.size();
        std::vector<int> perm(rank);
        auto it = n.iattrs.find("perm");
        for (int d = 0; d < rank; ++d) perm[d] = it == n.iattrs.end() ? rank - 1 - d : (int)it->second[d];
        if (it != n.iattrs.end() && (int)it->second.size() != rank) {
            set_error("Transpose: perm of length %zu for a rank-%d input", it->second.size(), rank);
            return ICX_ERR_SHAPE;
        }
        std::vector<int64_t> oshape(rank);
        for (int d = 0; d < rank; ++d) {
            if (perm[d] < 0 || perm[d] >= rank) {
                set_error("Transpose: perm is not a permutation");
                return ICX_ERR_INVALID_ARG;
            }
            oshape[d] = X->shape[perm[d]];
        }
        const std::vector<int64_t> ishape = X->shape;
        const void* x = X->ptr;
        const int dt = X->dtype;
        DevTensor* Y;
        rc = alloc(n.out[0], dt, oshape, &Y);
        if (rc) return rc;
        return icx_transpose(s_, x, dtype_size(dt), rank, ishape.data(), perm.data(), Y->ptr);
    }

    // Reshape: the output names the input's buffer with a new shape (no copy).
    int run_reshape(const Node& n) {
        if (n.in.size() != 2) {
            set_error("Reshape requires 2 inputs, got %zu", n.in.size());
            return ICX_ERR_INVALID_ARG;
        }
        std::vector<int64_t> xs, spec, tgt;
        int xdt;
        if (!shape_of(n.in[0], &xs, &xdt)) {
            set_error("Reshape: input tensor '%s' is missing", n.in[0].c_str());
            return ICX_ERR_INVALID_ARG;
        }
        int rc = host_ints(n.in[1], &spec, "Reshape");
        if (!rc) rc = reshape_target(xs, spec, n.attr_or("allowzero", 0) != 0, &tgt);
        if (rc) return rc;
        const HostTensor* h = host_known(n.in[0]);
        if (h && int_dtype(h->dtype)) {
            HostTensor t = *h;
            t.shape = tgt;
            return set_host(n.out[0], std::move(t));
        }
        const DevTensor* X;
        rc = need(n.in[0], &X, "Reshape");
        if (rc) return rc;
        DevTensor t = *X;
        t.shape = tgt;
        t.pooled = false;  // the buffer belongs to the input (kept alive by its last use)
        g_.values[n.out[0]] = t;
        return ICX_OK;
    }

    // f32 MatMul with the reference's batch rules (src/operators/matmul.rs:60-90).
    int run_matmul_f32(const Node& n) {
        const DevTensor *A, *B;
        int rc = need_f32(n.in[0], &A, "MatMul");
        if (!rc) rc = need_f32(n.in[1], &B, "MatMul");
        if (rc) return rc;
        if (A->shape.size() < 2 || B->shape.size() < 2) {
            set_error("MatMul: 1-D operands are not on this path (%s x %s)", shape_str(A->shape).c_str(),
                      shape_str(B->shape).c_str());
            return ICX_ERR_UNSUPPORTED;
        }
        const int64_t M = A->shape[A->shape.size() - 2], K = A->shape.back();
        const int64_t Kb = B->shape[B->shape.size() - 2], N = B->shape.back();
        if (K != Kb) {
            set_error("MatMul: inner dimensions must match: %lld != %lld", (long long)K, (long long)Kb);
            return ICX_ERR_SHAPE;
        }
        const std::vector<int64_t> ab(A->shape.begin(), A->shape.end() - 2), bb(B->shape.begin(), B->shape.end() - 2);
        std::vector<int64_t> ob;
        int b_bcast = 0;
        bool a_bcast = false;
        if (ab.empty() && !bb.empty()) {
            ob = bb;
            a_bcast = true;
        } else if (!ab.empty() && bb.empty()) {
            ob = ab;
            b_bcast = 1;
        } else if (ab == bb) {
            ob = ab;
        } else {
            set_error("MatMul: batch dimensions must be compatible for broadcasting: %s vs %s",
                      shape_str(ab).c_str(), shape_str(bb).c_str());
            return ICX_ERR_SHAPE;
        }
        if (a_bcast) {
            set_error("MatMul: a 2-D left operand with a batched right operand is not on this path");
            return ICX_ERR_UNSUPPORTED;
        }
        std::vector<int64_t> oshape = ob;
        oshape.push_back(M);
        oshape.push_back(N);
        const float *a = static_cast<const float*>(A->ptr), *b = static_cast<const float*>(B->ptr);
        DevTensor* C;
        rc = alloc(n.out[0], ICX_F32, oshape, &C);
        if (rc) return rc;
        return icx_matmul_f32(s_, a, b, (size_t)numel(ob), b_bcast, M, K, N, static_cast<float*>(C->ptr));
    }

    int run_matmul_integer(const Node& n) {
        if (n.in.size() < 2 || n.in.size() > 4) {
            set_error("MatMulInteger requires 2, 3, or 4 inputs, got %zu", n.in.size());
            return ICX_ERR_INVALID_ARG;
        }
        const DevTensor* A;
        int rc = need(n.in[0], &A, "MatMulInteger");
        if (rc) return rc;
        int64_t Kb, N;
        int b_dt, b_packed = 0;
        const void* b_ptr;
        const int32_t* colsum = nullptr;
        auto pk = g_.packed.find(n.in[1]);
        if (pk != g_.packed.end()) {
            Kb = pk->second.K;
            N = pk->second.N;
            b_dt = pk->second.dtype;
            b_ptr = pk->second.packed;
            colsum = pk->second.colsum;
            b_packed = 1;
        } else {
            const DevTensor* B;
            rc = need(n.in[1], &B, "MatMulInteger");
            if (rc) return rc;
            if (B->shape.size() != 2) {
                set_error("MatMulInteger: b must be 2-D, got %s", shape_str(B->shape).c_str());
                return ICX_ERR_SHAPE;
            }
            if (B->dtype != ICX_U8 && B->dtype != ICX_I8) {
                set_error("MatMulInteger: b dtype %s unsupported (must be Int8 or UInt8)", dtype_name(B->dtype));
                return ICX_ERR_DTYPE;
            }
            Kb = B->shape[0];
            N = B->shape[1];
            b_dt = B->dtype;
            b_ptr = B->ptr;
        }
        int64_t M;
        std::vector<int64_t> oshape;
        rc = gemm_rows(A, Kb, &M, &oshape);
        if (rc) return rc;
        oshape.push_back(N);
        const void *azp, *bzp;
        size_t alen, blen;
        rc = zero_point(n.in.size() > 2 ? n.in[2] : "", A->dtype, false, N, &azp, &alen);
        if (rc) return rc;
        rc = zero_point(n.in.size() > 3 ? n.in[3] : "", b_dt, true, N, &bzp, &blen);
        if (rc) return rc;
        const void* a_ptr = A->ptr;
        const int a_dt = A->dtype;
        DevTensor* C;
        rc = alloc(n.out[0], ICX_I32, oshape, &C);
        if (rc) return rc;
        rc = workspace(icx_matmul_integer_workspace_size(M, Kb, N, b_packed));
        if (rc) return rc;
        return icx_matmul_integer(s_, a_ptr, a_dt, b_ptr, b_dt, b_packed, colsum, M, Kb, N, azp, bzp, blen,
                                  nullptr, static_cast<int32_t*>(C->ptr), g_.ws, g_.ws_bytes);
    }

    int run_dql(const Node& n, bool from_head = false) {
        if (n.in.size() != 1 || n.out.size() != 3) {
            set_error("DynamicQuantizeLinear: expected 1 input and 3 outputs, got %zu and %zu", n.in.size(),
                      n.out.size());
            return ICX_ERR_INVALID_ARG;
        }
        if (g_.dql_done.count(n.out[0])) return ICX_OK;  // its producer's GEMM wrote y, scale, zp
        if (!from_head && g_.qin_dql.count(n.name)) return ICX_OK;  // its reader's launch runs it
        const DevTensor* X;
        int rc = need(n.in[0], &X, "DynamicQuantizeLinear");
        if (rc) return rc;
        if (X->dtype != ICX_F32) {
            set_error("DynamicQuantizeLinear: input must be Float32, got %s", dtype_name(X->dtype));
            return ICX_ERR_DTYPE;
        }
        const std::vector<int64_t> shape = X->shape;
        const float* x = static_cast<const float*>(X->ptr);
        const int64_t cnt = numel(shape);
        DevTensor *Y, *S, *Z, *R = nullptr;
        rc = alloc(n.out[0], ICX_U8, shape, &Y);
        if (!rc) rc = alloc(n.out[1], ICX_F32, {}, &S);
        if (!rc) rc = alloc(n.out[2], ICX_U8, {}, &Z);
        if (rc) return rc;
        size_t row_len = 0;
        if (g_.rowsum_wanted.count(n.out[0]) && !shape.empty() && shape.back() > 0) {
            row_len = (size_t)shape.back();
            const std::string rname = n.out[0] + "::rowsum";
            rc = alloc(rname, ICX_I32, {cnt / (int64_t)row_len}, &R);
            if (rc) return rc;
            g_.rowsum_of[n.out[0]] = rname;
        }
        auto rg = g_.range_of.find(n.in[0]);
        if (rg != g_.range_of.end() && cnt > 0) {  // the producer left the range: quantize only
            const DevTensor* P = find(rg->second.first);
            if (P)
                return icx::dql_from_parts(s_, x, cnt, static_cast<uint8_t*>(Y->ptr), static_cast<float*>(S->ptr),
                                           static_cast<uint8_t*>(Z->ptr), R ? static_cast<int32_t*>(R->ptr) : nullptr,
                                           row_len, static_cast<const float2*>(P->ptr), rg->second.second);
        }
        if (!R && g_.qsync && cnt > 0) {  // one launch, the blocks trading ranges through qsync
            rc = icx::dql_exchange(s_, x, cnt, static_cast<uint8_t*>(Y->ptr), static_cast<float*>(S->ptr),
                                   static_cast<uint8_t*>(Z->ptr), g_.qsync);
            if (rc == ICX_OK) {
                ++g_.dql_single;
                return ICX_OK;
            }
            if (rc != ICX_ERR_UNSUPPORTED) return rc;
            icx::clear_error();  // too large or unaligned: the two-launch path
        }
        rc = workspace(icx_dql_workspace_size(cnt));
        if (rc) return rc;
        return icx::dql_two_launch(s_, x, cnt, static_cast<uint8_t*>(Y->ptr), static_cast<float*>(S->ptr),
                                   static_cast<uint8_t*>(Z->ptr), R ? static_cast<int32_t*>(R->ptr) : nullptr,
                                   row_len, g_.ws, g_.ws_bytes, false);
    }

    // ReduceMean (src/operators/reduce_mean.rs:19-105): axes from the second input (opset 18)
    // or the `axes` attribute (earlier opsets; the reference's CPU forward reads the input
    // only, its GPU dispatch always reduces the last axis, src/cuda/executor/reduction.rs:
    // 88-104); none, or an empty list, reduces every element (data.mean()).  keepdims
    // (default 1) keeps the reduced axis as 1 — for the full reduction every axis, as ONNX
    // defines it (the reference's CPU forward returns a rank-0 tensor there, same value).  The
    // reference reduces only axes[0] of a longer list; more than one axis is refused here.
    int run_reduce_mean(const Node& n) {
        const DevTensor* X;
        int rc = need_f32(n.in[0], &X, "ReduceMean");
        if (rc) return rc;
        std::vector<int64_t> axes;
        if (n.in.size() > 1 && !n.in[1].empty()) {
            rc = host_ints(n.in[1], &axes, "ReduceMean");
            if (rc) return rc;
        } else {
            auto it = n.iattrs.find("axes");
            if (it != n.iattrs.end()) axes = it->second;
        }
        const std::vector<int64_t> shape = X->shape;
        const int r = (int)shape.size();
        const bool keep = n.attr_or("keepdims", 1) != 0;
        size_t outer = 1, len = (size_t)numel(shape), inner = 1;
        int seq = 0;
        std::vector<int64_t> oshape;
        if (axes.empty()) {
            if (keep) oshape.assign(r, 1);
        } else {
            if (axes.size() > 1) {
                set_error("ReduceMean: %zu axes; one axis is on this path", axes.size());
                return ICX_ERR_UNSUPPORTED;
            }
            const int64_t a = axes[0] < 0 ? axes[0] + r : axes[0];
            if (a < 0 || a >= r) {
                set_error("ReduceMean: axis %lld out of range for rank %d", (long long)axes[0], r);
                return ICX_ERR_SHAPE;
            }
            for (int64_t d = 0; d < a; ++d) outer *= (size_t)shape[d];
            len = (size_t)shape[a];
            for (int64_t d = a + 1; d < r; ++d) inner *= (size_t)shape[d];
            seq = a != r - 1;  // ndarray sums the last (least-strided) axis unrolled, others in order
            oshape = shape;
            if (keep) oshape[a] = 1;
            else oshape.erase(oshape.begin() + a);
        }
        if (len == 0 && outer * inner) {
            set_error("ReduceMean: the reduced axis of %s is empty", shape_str(shape).c_str());
            return ICX_ERR_SHAPE;
        }
        const float* x = static_cast<const float*>(X->ptr);
        DevTensor* Y;
        rc = alloc(n.out[0], ICX_F32, oshape, &Y);
        if (rc) return rc;
        return icx_reduce_mean_f32(s_, x, outer, len, inner, seq, static_cast<float*>(Y->ptr));
    }

    // Pow (src/operators/pow.rs:18-45): the exponent broadcasts over the base, whose shape the
    // output keeps (the reference's .broadcast(base.raw_dim()) panics otherwise).
    int run_pow(const Node& n) {
        if (n.in.size() != 2 || n.out.size() != 1) {
            set_error("Pow: expected 2 inputs and 1 output");
            return ICX_ERR_INVALID_ARG;
        }
        const DevTensor *X, *E;
        int rc = need_f32(n.in[0], &X, "Pow");
        if (!rc) rc = need_f32(n.in[1], &E, "Pow");
        if (rc) return rc;
        const int kind = bcast_kind(E->shape, X->shape);
        if (kind < 0) {
            set_error("Pow: exponent %s does not broadcast over the base %s", shape_str(E->shape).c_str(),
                      shape_str(X->shape).c_str());
            return ICX_ERR_SHAPE;
        }
        const std::vector<int64_t> shape = X->shape;
        const int64_t cols = shape.empty() ? 1 : shape.back();
        const int64_t rows = cols ? numel(shape) / cols : 0;
        const float *x = static_cast<const float*>(X->ptr), *e = static_cast<const float*>(E->ptr);
        DevTensor* Y;
        rc = alloc(n.out[0], ICX_F32, shape, &Y);
        if (rc) return rc;
        return icx_pow_f32(s_, x, (size_t)rows, (size_t)cols, e, kind, static_cast<float*>(Y->ptr));
    }

    int run_sqrt(const Node& n) {
        const DevTensor* X;
        int rc = need_f32(n.in[0], &X, "Sqrt");
        if (rc) return rc;
        const std::vector<int64_t> shape = X->shape;
        const float* x = static_cast<const float*>(X->ptr);
        DevTensor* Y;
        rc = alloc(n.out[0], ICX_F32, shape, &Y);
        if (rc) return rc;
        return icx_sqrt_f32(s_, x, (size_t)numel(shape), static_cast<float*>(Y->ptr));
    }

    int run_chain(const std::string& in_name, const std::vector<Step>& steps, const std::string& out_name,
                  const char* who) {
        const DevTensor* X;
        int rc = need_f32(in_name, &X, who);
        if (rc) return rc;
        const std::vector<int64_t> shape = X->shape;
        const float* x = static_cast<const float*>(X->ptr);
        const int64_t cols = shape.empty() ? 1 : shape.back();
        const int64_t rows = cols ? numel(shape) / cols : 0;
        icx_chain ch;
        rc = make_chain(steps, shape, ch, who);
        if (rc) return rc;
        DevTensor* Y;
        rc = alloc(out_name, ICX_F32, shape, &Y);
        if (rc) return rc;
        return icx_fused_chain_f32(s_, x, rows, cols, &ch, static_cast<float*>(Y->ptr));
    }

    // Mul / Add / Sub / Div outside a chain: the chain kernel when the output has one
    // operand's shape and the other broadcasts as a chain operand, else a general broadcast
    // kernel; integer operands known on the host are shape arithmetic, done on the host.
    int run_binary(const Node& n) {
        if (n.in.size() != 2 || n.out.size() != 1) {
            set_error("%s: expected 2 inputs and 1 output", n.op.c_str());
            return ICX_ERR_INVALID_ARG;
        }
        std::vector<const HostTensor*> hs;
        if (all_host(n, 2, &hs)) {
            int rc = host_binary(n, *hs[0], *hs[1]);
            if (rc != kHostTooLarge) return rc;
        }
        return binary_f32_into(op_code(n.op), n.in[0], n.in[1], n.out[0], n.op.c_str());
    }

    // out = a op b on Float32 device tensors: the chain kernel when the output has one
    // operand's shape and the other broadcasts as a chain operand, else the general
    // broadcast kernel (e.g. [1, S, D] over [B, S, D]).
    int binary_f32_into(int op, const std::string& an, const std::string& bn, const std::string& outn,
                        const char* who) {
        const DevTensor *A, *B;
        int rc = need(an, &A, who);
        if (!rc) rc = need(bn, &B, who);
        if (rc) return rc;
        bool ok;
        const std::vector<int64_t> out = broadcast_shape(A->shape, B->shape, &ok);
        if (!ok) {
            set_error("%s: shapes %s and %s do not broadcast", who, shape_str(A->shape).c_str(),
                      shape_str(B->shape).c_str());
            return ICX_ERR_SHAPE;
        }
        if (A->dtype != ICX_F32 || B->dtype != ICX_F32) {
            set_error("%s: device operands of dtypes %s and %s (Float32 only; integer arithmetic runs on host-known "
                      "shape tensors)", who, dtype_name(A->dtype), dtype_name(B->dtype));
            return ICX_ERR_DTYPE;
        }
        Step st;
        st.op = op;
        if (A->shape == out && bcast_kind(B->shape, out) >= 0) {
            st.opnd0 = bn;
            return run_chain(an, {st}, outn, who);
        }
        if (B->shape == out && bcast_kind(A->shape, out) >= 0) {
            st.lhs = true;
            st.opnd0 = an;
            return run_chain(bn, {st}, outn, who);
        }
        const std::vector<int64_t> ast = bcast_strides(A->shape, out), bst = bcast_strides(B->shape, out);
        const float *a = static_cast<const float*>(A->ptr), *b = static_cast<const float*>(B->ptr);
        DevTensor* Y;
        rc = alloc(outn, ICX_F32, out, &Y);
        if (rc) return rc;
        return icx::binary_f32(s_, op, a, ast.data(), b, bst.data(), (int)out.size(), out.data(),
                               static_cast<float*>(Y->ptr));
    }

    // Cast (src/operators/cast.rs; GPU dispatch src/cuda/executor/layout.rs:148-172) to
    // FLOAT / INT32 / INT64 / BOOL, with Rust's `as` semantics.
    int run_cast(const Node& n) {
        const int64_t to = n.attr_or("to", -1);
        int dst;
        switch (to) {
            case 1: dst = ICX_F32; break;
            case 6: dst = ICX_I32; break;
            case 7: dst = ICX_I64; break;
            case 9: dst = ICX_BOOL; break;
            default:
                set_error("Cast to ONNX dtype %lld is not on this path (FLOAT, INT32, INT64, BOOL)", (long long)to);
                return ICX_ERR_UNSUPPORTED;
        }
        std::vector<const HostTensor*> hs;
        if (all_host(n, 1, &hs)) {
            const HostTensor& x = *hs[0];
            HostTensor y = host_tensor(dst, x.shape);
            const int64_t cnt = numel(x.shape);
            for (int64_t i = 0; i < cnt; ++i) {  // integer / Bool source (all_host)
                const int64_t v = int_at(x, i);
                if (dst == ICX_F32) reinterpret_cast<float*>(y.data.data())[i] = (float)v;  // RNE
                else put_int(y, i, v);
            }
            return set_host(n.out[0], std::move(y));
        }
        const DevTensor* X;
        int rc = need(n.in[0], &X, "Cast");
        if (rc) return rc;
        const std::vector<int64_t> shape = X->shape;
        const void* x = X->ptr;
        const int src = X->dtype;
        const size_t cnt = (size_t)numel(shape);
        DevTensor* Y;
        rc = alloc(n.out[0], dst, shape, &Y);
        if (rc) return rc;
        if (src == dst) {
            if (cnt) ICX_HIP_CHECK(hipMemcpyAsync(Y->ptr, x, cnt * dtype_size(dst), hipMemcpyDeviceToDevice, s_));
            return ICX_OK;
        }
        if (src == ICX_I32 && dst == ICX_F32)
            return icx_cast_i32_f32(s_, static_cast<const int32_t*>(x), cnt, static_cast<float*>(Y->ptr));
        return icx::cast_any(s_, src, x, dst, Y->ptr, cnt);
    }

    // DequantizeLinear (src/operators/dequantize_linear.rs:32-180): per-tensor or per-axis.
    // Gather (src/cuda/executor/layout.rs:260-330 -> gpu_gather_from_gpu; CPU
    // src/operators/gather.rs:21-205): any axis, data of any dtype on this path (the UINT8
    // embedding table of DistilBERT-INT8 first of all), Int64 or Int32 indices; the output
    // keeps the data dtype, as the GPU path does.
    int run_gather(const Node& n) {
        if (n.in.size() != 2 || n.out.size() != 1) {
            set_error("Gather requires [data, indices] and one output");
            return ICX_ERR_INVALID_ARG;
        }
        std::vector<const HostTensor*> hs;
        if (all_host(n, 2, &hs)) {
            int rc = host_gather(n, *hs[0], *hs[1]);
            if (rc != kHostTooLarge) return rc;
        }
        const DevTensor *D, *I;
        int rc = need(n.in[0], &D, "Gather");
        if (!rc) rc = need(n.in[1], &I, "Gather");
        if (rc) return rc;
        if (I->dtype != ICX_I64 && I->dtype != ICX_I32) {
            set_error("Gather: indices must be Int64 or Int32, got %s", dtype_name(I->dtype));
            return ICX_ERR_DTYPE;
        }
        const int64_t nd = (int64_t)D->shape.size();
        const int64_t ax0 = n.attr_or("axis", 0);
        const int64_t ax = ax0 < 0 ? ax0 + nd : ax0;
        if (nd < 1 || ax < 0 || ax >= nd) {
            set_error("Gather: axis %lld out of range for rank-%lld data", (long long)ax0, (long long)nd);
            return ICX_ERR_SHAPE;
        }
        int64_t outer = 1, inner = 1;
        for (int64_t d = 0; d < ax; ++d) outer *= D->shape[d];
        for (int64_t d = ax + 1; d < nd; ++d) inner *= D->shape[d];
        std::vector<int64_t> oshape(D->shape.begin(), D->shape.begin() + ax);
        oshape.insert(oshape.end(), I->shape.begin(), I->shape.end());
        oshape.insert(oshape.end(), D->shape.begin() + ax + 1, D->shape.end());
        const int dt = D->dtype;
        const void* dptr = D->ptr;
        const void* iptr = I->ptr;
        const int idt = I->dtype;
        const size_t nidx = (size_t)numel(I->shape);
        const int64_t alen = D->shape[ax];
        DevTensor* Y;
        rc = alloc(n.out[0], dt, oshape, &Y);
        if (rc) return rc;
        return icx_gather(s_, dptr, dtype_size(dt), (size_t)outer, (size_t)alen, (size_t)inner, iptr, idt, nidx,
                          Y->ptr);
    }

    int run_dequantize(const Node& n) {
        if (n.in.size() < 2 || n.in.size() > 3) {
            set_error("DequantizeLinear requires 2 or 3 inputs, got %zu", n.in.size());
            return ICX_ERR_INVALID_ARG;
        }
        const DevTensor *X, *S, *Z = nullptr;
        int rc = need(n.in[0], &X, "DequantizeLinear");
        if (!rc) rc = need(n.in[1], &S, "DequantizeLinear");
        if (!rc && n.in.size() == 3 && !n.in[2].empty()) rc = need(n.in[2], &Z, "DequantizeLinear");
        if (rc) return rc;
        if (S->dtype != ICX_F32) {
            set_error("DequantizeLinear: x_scale must be Float32, got %s", dtype_name(S->dtype));
            return ICX_ERR_DTYPE;
        }
        const int64_t cnt = numel(X->shape);
        const int64_t slen = numel(S->shape);
        int64_t axis_size = 1, inner = std::max<int64_t>(cnt, 1);
        if (!(S->shape.empty() || (S->shape.size() == 1 && slen == 1))) {
            const int64_t nd = (int64_t)X->shape.size();
            const int64_t ax0 = n.attr_or("axis", 1);
            const int64_t ax = ax0 < 0 ? ax0 + nd : ax0;
            if (ax < 0 || ax >= nd) {
                set_error("DequantizeLinear: axis %lld out of range for a rank-%lld input", (long long)ax0,
                          (long long)nd);
                return ICX_ERR_SHAPE;
            }
            axis_size = X->shape[ax];
            if (S->shape.size() != 1 || slen != axis_size) {
                set_error("DequantizeLinear: per-axis scale of shape %s does not match input dim %lld (%lld)",
                          shape_str(S->shape).c_str(), (long long)ax, (long long)axis_size);
                return ICX_ERR_SHAPE;
            }
            inner = 1;
            for (int64_t d = ax + 1; d < nd; ++d) inner *= X->shape[d];
        }
        if (Z) {
            if (Z->dtype != X->dtype) {
                set_error("DequantizeLinear: x_zero_point dtype %s must match x dtype %s", dtype_name(Z->dtype),
                          dtype_name(X->dtype));
                return ICX_ERR_DTYPE;
            }
            if (numel(Z->shape) != slen) {
                set_error("DequantizeLinear: x_zero_point shape %s must match x_scale shape %s",
                          shape_str(Z->shape).c_str(), shape_str(S->shape).c_str());
                return ICX_ERR_SHAPE;
            }
        }
        const std::vector<int64_t> shape = X->shape;
        const void *x = X->ptr, *zp = Z ? Z->ptr : nullptr;
        const float* sc = static_cast<const float*>(S->ptr);
        const int x_dt = X->dtype;
        DevTensor* Y;
        rc = alloc(n.out[0], ICX_F32, shape, &Y);
        if (rc) return rc;
        return icx_dequantize_linear_f32(s_, x, x_dt, sc, zp, cnt, axis_size, inner, static_cast<float*>(Y->ptr));
    }

    // ---- the shape / mask plumbing of an exported encoder ----------------------------------
    // Shape (src/operators/shape.rs; GPU layout.rs:136-146): always on the host, Int64 [n],
    // with opset 15's start / end clamped as the reference does.
    int run_shape(const Node& n) {
        std::vector<int64_t> xs;
        int xdt;
        if (n.in.empty() || !shape_of(n.in[0], &xs, &xdt)) {
            set_error("Shape: input tensor '%s' is missing", n.in.empty() ? "" : n.in[0].c_str());
            return ICX_ERR_INVALID_ARG;
        }
        const int64_t r = (int64_t)xs.size();
        const int64_t s0 = n.attr_or("start", 0);
        const int64_t start = s0 < 0 ? std::max<int64_t>(r + s0, 0) : std::min(s0, r);
        int64_t end = r;
        if (n.attr.count("end")) {
            const int64_t e0 = n.attr.at("end");
            end = e0 < 0 ? std::max<int64_t>(r + e0, 0) : std::min(e0, r);
        }
        end = std::max(end, start);
        HostTensor t = host_tensor(ICX_I64, {end - start});
        for (int64_t i = start; i < end; ++i) put_int(t, i - start, xs[(size_t)i]);
        return set_host(n.out[0], std::move(t));
    }

    // Unsqueeze / Squeeze / Identity (GPU layout.rs:579-662): a new shape over the same
    // elements — a view of a device tensor (as Reshape), a copy of a host one.  Axes come
    // from the input (opset 13) or the attribute, negative ones counted from the output rank
    // (Unsqueeze) or the input rank (Squeeze); Squeeze without axes drops every unit dim, and
    // with axes drops the listed ones that are 1.
    int run_view(const Node& n) {
        std::vector<int64_t> xs;
        int xdt;
        if (n.in.empty() || !shape_of(n.in[0], &xs, &xdt)) {
            set_error("%s: input tensor '%s' is missing", n.op.c_str(), n.in.empty() ? "" : n.in[0].c_str());
            return ICX_ERR_INVALID_ARG;
        }
        std::vector<int64_t> oshape, axes;
        bool have = false;
        if (n.in.size() > 1 && !n.in[1].empty()) {
            int rc = host_ints(n.in[1], &axes, n.op.c_str());
            if (rc) return rc;
            have = true;
        } else if (n.iattrs.count("axes")) {
            axes = n.iattrs.at("axes");
            have = true;
        }
        if (n.op == "Identity") {
            oshape = xs;
        } else if (n.op == "Unsqueeze") {
            if (!have) {
                set_error("Unsqueeze requires an 'axes' attribute or input");
                return ICX_ERR_INVALID_ARG;
            }
            const int64_t r = (int64_t)(xs.size() + axes.size());
            std::vector<char> ins((size_t)r, 0);
            for (int64_t a : axes) {
                const int64_t ax = a < 0 ? a + r : a;
                if (ax < 0 || ax >= r || ins[(size_t)ax]) {
                    set_error("Unsqueeze: axis %lld is out of range or repeated for output rank %lld", (long long)a,
                              (long long)r);
                    return ICX_ERR_SHAPE;
                }
                ins[(size_t)ax] = 1;
            }
            size_t k = 0;
            for (int64_t d = 0; d < r; ++d) oshape.push_back(ins[(size_t)d] ? 1 : xs[k++]);
        } else {  // Squeeze
            const int64_t r = (int64_t)xs.size();
            std::vector<char> drop((size_t)r, have ? 0 : 1);
            for (int64_t a : axes) {
                const int64_t ax = a < 0 ? a + r : a;
                if (ax < 0 || ax >= r) {
                    set_error("Squeeze: axis %lld out of range for rank %lld", (long long)a, (long long)r);
                    return ICX_ERR_SHAPE;
                }
                drop[(size_t)ax] = 1;
            }
            for (int64_t d = 0; d < r; ++d)
                if (!(drop[(size_t)d] && xs[(size_t)d] == 1)) oshape.push_back(xs[(size_t)d]);
        }
        const HostTensor* h = host_known(n.in[0]);
        if (h && int_dtype(h->dtype)) {
            HostTensor t = *h;
            t.shape = oshape;
            return set_host(n.out[0], std::move(t));
        }
        const DevTensor* X;
        int rc = need(n.in[0], &X, n.op.c_str());
        if (rc) return rc;
        DevTensor t = *X;
        t.shape = oshape;
        t.pooled = false;  // the buffer belongs to the input
        g_.values[n.out[0]] = t;
        return ICX_OK;
    }

    // Concat (src/operators/concat.rs; GPU gpu_concat via layout.rs:664-667): one strided
    // copy per non-empty input into its slot of the output.
    int run_concat(const Node& n) {
        if (n.in.empty() || n.out.size() != 1) {
            set_error("Concat requires at least one input and one output");
            return ICX_ERR_INVALID_ARG;
        }
        std::vector<std::vector<int64_t>> shapes(n.in.size());
        int dt = -1;
        for (size_t i = 0; i < n.in.size(); ++i) {
            int d;
            if (!shape_of(n.in[i], &shapes[i], &d)) {
                set_error("Concat: input tensor '%s' is missing", n.in[i].c_str());
                return ICX_ERR_INVALID_ARG;
            }
            if (i && d != dt) {
                set_error("Concat: inputs of dtypes %s and %s", dtype_name(dt), dtype_name(d));
                return ICX_ERR_DTYPE;
            }
            dt = d;
        }
        const int64_t r = (int64_t)shapes[0].size();
        const int64_t a0 = n.attr_or("axis", 0);
        const int64_t ax = a0 < 0 ? a0 + r : a0;
        if (ax < 0 || ax >= r) {
            set_error("Concat: axis %lld out of range for rank %lld", (long long)a0, (long long)r);
            return ICX_ERR_SHAPE;
        }
        std::vector<int64_t> oshape = shapes[0];
        oshape[(size_t)ax] = 0;
        for (auto& sh : shapes) {
            bool ok = (int64_t)sh.size() == r;
            for (int64_t d = 0; ok && d < r; ++d) ok = d == ax || sh[(size_t)d] == shapes[0][(size_t)d];
            if (!ok) {
                set_error("Concat: input shape %s does not match %s off axis %lld", shape_str(sh).c_str(),
                          shape_str(shapes[0]).c_str(), (long long)ax);
                return ICX_ERR_SHAPE;
            }
            oshape[(size_t)ax] += sh[(size_t)ax];
        }
        const std::vector<int64_t> ost = dense_strides(oshape);
        std::vector<const HostTensor*> hs;
        if (all_host(n, n.in.size(), &hs) && numel(oshape) <= kHostFoldMax) {
            HostTensor y = host_tensor(dt, oshape);
            const size_t es = dtype_size(dt);
            int64_t at = 0;
            for (size_t i = 0; i < n.in.size(); ++i) {
                const std::vector<int64_t> ist = dense_strides(shapes[i]);
                for_each_offset(shapes[i], {ost, ist}, {at * ost[(size_t)ax], 0}, [&](int64_t, const std::vector<int64_t>& o) {
                    std::memcpy(&y.data[(size_t)o[0] * es], &hs[i]->data[(size_t)o[1] * es], es);
                });
                at += shapes[i][(size_t)ax];
            }
            return set_host(n.out[0], std::move(y));
        }
        std::vector<const DevTensor*> xs(n.in.size());
        for (size_t i = 0; i < n.in.size(); ++i) {
            int rc = need(n.in[i], &xs[i], "Concat");
            if (rc) return rc;
        }
        std::vector<const void*> ptrs;
        for (auto* x : xs) ptrs.push_back(x->ptr);
        DevTensor* Y;
        int rc = alloc(n.out[0], dt, oshape, &Y);
        if (rc) return rc;
        int64_t at = 0;
        for (size_t i = 0; i < n.in.size(); ++i) {
            const std::vector<int64_t> ist = dense_strides(shapes[i]);
            rc = icx::strided_copy(s_, ptrs[i], Y->ptr, dtype_size(dt), (int)r, shapes[i].data(), ist.data(), 0,
                                   ost.data(), at * ost[(size_t)ax]);
            if (rc) return rc;
            at += shapes[i][(size_t)ax];
        }
        return ICX_OK;
    }

    // Slice (GPU gpu_slice_nd via layout.rs:345-456; CPU src/operators/slice.rs): starts /
    // ends / axes / steps read on the host, one strided copy.
    int run_slice(const Node& n) {
        if (n.in.size() < 3 || n.out.size() != 1) {
            set_error("Slice requires at least 3 inputs: data, starts, ends");
            return ICX_ERR_INVALID_ARG;
        }
        std::vector<int64_t> xs, starts, ends, axes, steps, first, step, len;
        int dt;
        if (!shape_of(n.in[0], &xs, &dt)) {
            set_error("Slice: input tensor '%s' is missing", n.in[0].c_str());
            return ICX_ERR_INVALID_ARG;
        }
        int rc = host_ints(n.in[1], &starts, "Slice");
        if (!rc) rc = host_ints(n.in[2], &ends, "Slice");
        const bool has_axes = n.in.size() > 3 && !n.in[3].empty(), has_steps = n.in.size() > 4 && !n.in[4].empty();
        if (!rc && has_axes) rc = host_ints(n.in[3], &axes, "Slice");
        if (!rc && has_steps) rc = host_ints(n.in[4], &steps, "Slice");
        if (!rc)
            rc = slice_params(xs, starts, ends, has_axes ? &axes : nullptr, has_steps ? &steps : nullptr, &first, &step,
                              &len);
        if (rc) return rc;
        const std::vector<int64_t> ist = dense_strides(xs);
        std::vector<int64_t> xst(xs.size());
        int64_t x_off = 0;
        for (size_t d = 0; d < xs.size(); ++d) {
            xst[d] = step[d] * ist[d];
            if (len[d] > 0) x_off += first[d] * ist[d];
        }
        const std::vector<int64_t> ost = dense_strides(len);
        std::vector<const HostTensor*> hs;
        if (all_host(n, 1, &hs) && numel(len) <= kHostFoldMax) {
            HostTensor y = host_tensor(dt, len);
            const size_t es = dtype_size(dt);
            if (numel(len) > 0)
                for_each_offset(len, {ost, xst}, {0, x_off}, [&](int64_t, const std::vector<int64_t>& o) {
                    std::memcpy(&y.data[(size_t)o[0] * es], &hs[0]->data[(size_t)o[1] * es], es);
                });
            return set_host(n.out[0], std::move(y));
        }
        const DevTensor* X;
        rc = need(n.in[0], &X, "Slice");
        if (rc) return rc;
        const void* x = X->ptr;
        DevTensor* Y;
        rc = alloc(n.out[0], dt, len, &Y);
        if (rc) return rc;
        return icx::strided_copy(s_, x, Y->ptr, dtype_size(dt), (int)len.size(), len.data(), xst.data(), x_off,
                                 ost.data(), 0);
    }

    // Expand (GPU gpu_expand, src/cuda/ops/layout/mod.rs:1624-1670): bidirectional
    // broadcast of the input and the target shape, one strided copy with stride 0 on the
    // broadcast dimensions.
    int run_expand(const Node& n) {
        if (n.in.size() != 2 || n.out.size() != 1) {
            set_error("Expand requires [input, shape] and one output");
            return ICX_ERR_INVALID_ARG;
        }
        std::vector<int64_t> xs, target;
        int dt;
        if (!shape_of(n.in[0], &xs, &dt)) {
            set_error("Expand: input tensor '%s' is missing", n.in[0].c_str());
            return ICX_ERR_INVALID_ARG;
        }
        int rc = host_ints(n.in[1], &target, "Expand");
        if (rc) return rc;
        bool ok;
        const std::vector<int64_t> oshape = broadcast_shape(xs, target, &ok);
        if (!ok) {
            set_error("Expand: shapes %s and %s are not broadcastable", shape_str(xs).c_str(), shape_str(target).c_str());
            return ICX_ERR_SHAPE;
        }
        const std::vector<int64_t> xst = bcast_strides(xs, oshape), ost = dense_strides(oshape);
        std::vector<const HostTensor*> hs;
        if (all_host(n, 1, &hs) && numel(oshape) <= kHostFoldMax) {
            HostTensor y = host_tensor(dt, oshape);
            const size_t es = dtype_size(dt);
            for_each_offset(oshape, {ost, xst}, {0, 0}, [&](int64_t, const std::vector<int64_t>& o) {
                std::memcpy(&y.data[(size_t)o[0] * es], &hs[0]->data[(size_t)o[1] * es], es);
            });
            return set_host(n.out[0], std::move(y));
        }
        const DevTensor* X;
        rc = need(n.in[0], &X, "Expand");
        if (rc) return rc;
        const void* x = X->ptr;
        DevTensor* Y;
        rc = alloc(n.out[0], dt, oshape, &Y);
        if (rc) return rc;
        return icx::strided_copy(s_, x, Y->ptr, dtype_size(dt), (int)oshape.size(), oshape.data(), xst.data(), 0,
                                 ost.data(), 0);
    }

    // Equal (src/operators/equal.rs; GPU elementwise.rs:333): numpy broadcasting, Bool out.
    int run_equal(const Node& n) {
        if (n.in.size() != 2 || n.out.size() != 1) {
            set_error("Equal: expected 2 inputs and 1 output");
            return ICX_ERR_INVALID_ARG;
        }
        std::vector<int64_t> as, bs;
        int adt, bdt;
        if (!shape_of(n.in[0], &as, &adt) || !shape_of(n.in[1], &bs, &bdt)) {
            set_error("Equal: an input tensor is missing");
            return ICX_ERR_INVALID_ARG;
        }
        if (adt != bdt) {
            set_error("Equal: operands of dtypes %s and %s", dtype_name(adt), dtype_name(bdt));
            return ICX_ERR_DTYPE;
        }
        bool ok;
        const std::vector<int64_t> oshape = broadcast_shape(as, bs, &ok);
        if (!ok) {
            set_error("Equal: shapes %s and %s do not broadcast", shape_str(as).c_str(), shape_str(bs).c_str());
            return ICX_ERR_SHAPE;
        }
        const std::vector<int64_t> ast = bcast_strides(as, oshape), bst = bcast_strides(bs, oshape);
        std::vector<const HostTensor*> hs;
        if (all_host(n, 2, &hs) && numel(oshape) <= kHostFoldMax) {
            HostTensor y = host_tensor(ICX_BOOL, oshape);
            for_each_offset(oshape, {ast, bst}, {0, 0}, [&](int64_t e, const std::vector<int64_t>& o) {
                y.data[(size_t)e] = int_at(*hs[0], o[0]) == int_at(*hs[1], o[1]);
            });
            return set_host(n.out[0], std::move(y));
        }
        const DevTensor *A, *B;
        int rc = need(n.in[0], &A, "Equal");
        if (!rc) rc = need(n.in[1], &B, "Equal");
        if (rc) return rc;
        const void *a = A->ptr, *b = B->ptr;
        DevTensor* Y;
        rc = alloc(n.out[0], ICX_BOOL, oshape, &Y);
        if (rc) return rc;
        return icx::compare_equal(s_, adt, a, ast.data(), b, bst.data(), (int)oshape.size(), oshape.data(),
                                  static_cast<uint8_t*>(Y->ptr));
    }

    // Where (src/operators/where_op.rs; GPU layout.rs:62-134): three-way numpy broadcasting;
    // a condition that is not Bool is cast to Bool first, as the reference does.
    int run_where(const Node& n) {
        if (n.in.size() != 3 || n.out.size() != 1) {
            set_error("Where requires [condition, x, y] and one output");
            return ICX_ERR_INVALID_ARG;
        }
        std::vector<int64_t> cs, xs, ys;
        int cdt, xdt, ydt;
        if (!shape_of(n.in[0], &cs, &cdt) || !shape_of(n.in[1], &xs, &xdt) || !shape_of(n.in[2], &ys, &ydt)) {
            set_error("Where: an input tensor is missing");
            return ICX_ERR_INVALID_ARG;
        }
        if (xdt != ydt) {
            set_error("Where: x and y of dtypes %s and %s", dtype_name(xdt), dtype_name(ydt));
            return ICX_ERR_DTYPE;
        }
        bool ok1, ok2;
        const std::vector<int64_t> cx = broadcast_shape(cs, xs, &ok1);
        const std::vector<int64_t> oshape = broadcast_shape(cx, ys, &ok2);
        if (!ok1 || !ok2) {
            set_error("Where: shapes %s, %s and %s are not broadcastable", shape_str(cs).c_str(), shape_str(xs).c_str(),
                      shape_str(ys).c_str());
            return ICX_ERR_SHAPE;
        }
        const std::vector<int64_t> cst = bcast_strides(cs, oshape), xst = bcast_strides(xs, oshape),
                                   yst = bcast_strides(ys, oshape);
        const size_t es = dtype_size(xdt);
        std::vector<const HostTensor*> hs;
        if (all_host(n, 3, &hs) && numel(oshape) <= kHostFoldMax) {
            HostTensor y = host_tensor(xdt, oshape);
            for_each_offset(oshape, {cst, xst, yst}, {0, 0, 0}, [&](int64_t e, const std::vector<int64_t>& o) {
                const bool c = int_at(*hs[0], o[0]) != 0;
                std::memcpy(&y.data[(size_t)e * es], &(c ? hs[1] : hs[2])->data[(size_t)(c ? o[1] : o[2]) * es], es);
            });
            return set_host(n.out[0], std::move(y));
        }
        const DevTensor *C, *X, *Yv;
        int rc = need(n.in[0], &C, "Where");
        if (!rc) rc = need(n.in[1], &X, "Where");
        if (!rc) rc = need(n.in[2], &Yv, "Where");
        if (rc) return rc;
        const void* c = C->ptr;
        const void *x = X->ptr, *yv = Yv->ptr;
        if (cdt != ICX_BOOL && cdt != ICX_U8) {  // condition to Bool (x != 0)
            DevTensor* T;
            const size_t cnt = (size_t)numel(cs);
            rc = alloc(n.out[0] + "::cond", ICX_BOOL, cs, &T);
            if (!rc) rc = icx::cast_any(s_, cdt, c, ICX_BOOL, T->ptr, cnt);
            if (rc) return rc;
            c = T->ptr;
        }
        DevTensor* O;
        rc = alloc(n.out[0], xdt, oshape, &O);
        if (rc) return rc;
        return icx::select_where(s_, es, static_cast<const uint8_t*>(c), cst.data(), x, xst.data(), yv, yst.data(),
                                 (int)oshape.size(), oshape.data(), O->ptr);
    }

    // Gather of a host-known integer tensor (typically a Shape result) on the host, with the
    // index rules of icx_gather.
    int host_gather(const Node& n, const HostTensor& D, const HostTensor& I) const {
        if (I.dtype != ICX_I64 && I.dtype != ICX_I32) {
            set_error("Gather: indices must be Int64 or Int32, got %s", dtype_name(I.dtype));
            return ICX_ERR_DTYPE;
        }
        const int64_t nd = (int64_t)D.shape.size();
        const int64_t ax0 = n.attr_or("axis", 0);
        const int64_t ax = ax0 < 0 ? ax0 + nd : ax0;
        if (nd < 1 || ax < 0 || ax >= nd) {
            set_error("Gather: axis %lld out of range for rank-%lld data", (long long)ax0, (long long)nd);
            return ICX_ERR_SHAPE;
        }
        int64_t outer = 1, inner = 1;
        for (int64_t d = 0; d < ax; ++d) outer *= D.shape[(size_t)d];
        for (int64_t d = ax + 1; d < nd; ++d) inner *= D.shape[(size_t)d];
        std::vector<int64_t> oshape(D.shape.begin(), D.shape.begin() + ax);
        oshape.insert(oshape.end(), I.shape.begin(), I.shape.end());
        oshape.insert(oshape.end(), D.shape.begin() + ax + 1, D.shape.end());
        if (numel(oshape) > kHostFoldMax) return kHostTooLarge;
        const int64_t alen = D.shape[(size_t)ax], ni = numel(I.shape);
        if (alen == 0 && ni * outer * inner > 0) {
            set_error("Gather: %lld indices into an empty axis", (long long)ni);
            return ICX_ERR_SHAPE;
        }
        const size_t es = dtype_size(D.dtype);
        HostTensor y = host_tensor(D.dtype, oshape);
        for (int64_t o = 0; o < outer; ++o)
            for (int64_t j = 0; j < ni; ++j) {
                int64_t k = int_at(I, j);  // negative from the end, then clamped as icx_gather does
                if (k < 0) k += alen;
                k = std::min(std::max<int64_t>(k, 0), alen - 1);
                std::memcpy(&y.data[(size_t)((o * ni + j) * inner) * es], &D.data[(size_t)((o * alen + k) * inner) * es],
                            (size_t)inner * es);
            }
        return set_host(n.out[0], std::move(y));
    }

    // Add / Sub / Mul / Div of host-known integer tensors (shape arithmetic), numpy
    // broadcasting, wrapping as Rust's release build; integer division truncates, and
    // division by zero or of the minimum by -1 is an error (Rust panics).
    int host_binary(const Node& n, const HostTensor& A, const HostTensor& B) const {
        if (A.dtype != B.dtype || A.dtype == ICX_BOOL) {
            set_error("%s: operands of dtypes %s and %s", n.op.c_str(), dtype_name(A.dtype), dtype_name(B.dtype));
            return ICX_ERR_DTYPE;
        }
        bool ok;
        const std::vector<int64_t> oshape = broadcast_shape(A.shape, B.shape, &ok);
        if (!ok) {
            set_error("%s: shapes %s and %s do not broadcast", n.op.c_str(), shape_str(A.shape).c_str(),
                      shape_str(B.shape).c_str());
            return ICX_ERR_SHAPE;
        }
        if (numel(oshape) > kHostFoldMax) return kHostTooLarge;
        HostTensor y = host_tensor(A.dtype, oshape);
        const int op = op_code(n.op);
        const int64_t lo = A.dtype == ICX_I64 ? INT64_MIN : A.dtype == ICX_I32 ? INT32_MIN : A.dtype == ICX_I8 ? -128 : 0;
        int bad = 0;
        for_each_offset(oshape, {bcast_strides(A.shape, oshape), bcast_strides(B.shape, oshape)}, {0, 0},
                        [&](int64_t e, const std::vector<int64_t>& o) {
                            const int64_t a = int_at(A, o[0]), b = int_at(B, o[1]);
                            uint64_t r = 0;
                            switch (op) {
                                case ICX_OP_ADD: r = (uint64_t)a + (uint64_t)b; break;
                                case ICX_OP_SUB: r = (uint64_t)a - (uint64_t)b; break;
                                case ICX_OP_MUL: r = (uint64_t)a * (uint64_t)b; break;
                                default:
                                    if (b == 0 || (b == -1 && a == lo)) bad = 1;
                                    else r = (uint64_t)(a / b);
                            }
                            put_int(y, e, (int64_t)r);
                        });
        if (bad) {
            set_error("%s: integer division by zero or overflow", n.op.c_str());
            return ICX_ERR_INVALID_ARG;
        }
        return set_host(n.out[0], std::move(y));
    }

   public:
    // Outputs the caller asked for that exist only on the host this run: upload them.
    int finish_outputs() {
        for (auto& o : g_.live_outputs) {
            if (g_.values.count(o) || !g_.hv.count(o)) continue;
            const DevTensor* d;
            int rc = materialize(o, &d);
            if (rc) return rc;
        }
        return ICX_OK;
    }
};

std::vector<std::string> names_of(int n, const char* const* p) {
    std::vector<std::string> v;
    for (int i = 0; i < n; ++i) v.emplace_back(p && p[i] ? p[i] : "");
    return v;
}

bool valid_dtype(int dt) {
    return dt == ICX_I8 || dt == ICX_U8 || dt == ICX_I32 || dt == ICX_F32 || dt == ICX_BOOL;
}

}  // namespace

// ---------------------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------------------
extern "C" icx_graph* icx_graph_create(void) { return new (std::nothrow) icx_graph(); }

extern "C" void icx_graph_destroy(icx_graph* g) { delete g; }

extern "C" int icx_graph_add_input(icx_graph* g, const char* name, int rank, const int64_t* dims) {
    icx::clear_error();
    if (!g || !name || rank < 0 || (rank && !dims)) ICX_FAIL(ICX_ERR_INVALID_ARG, "add_input: bad arguments");
    g->inputs.emplace_back(name, std::vector<int64_t>(dims, dims + rank));
    g->invalidate();
    return ICX_OK;
}

extern "C" int icx_graph_add_initializer(icx_graph* g, const char* name, int dtype, int rank,
                                         const int64_t* dims, const void* host_data) {
    icx::clear_error();
    if (!g || !name || rank < 0 || (rank && !dims)) ICX_FAIL(ICX_ERR_INVALID_ARG, "add_initializer: bad arguments");
    if (!valid_dtype(dtype) && dtype != ICX_I64)
        ICX_FAIL(ICX_ERR_DTYPE, "add_initializer: '%s' has unsupported dtype %d", name, dtype);
    HostTensor t;
    t.dtype = dtype;
    t.shape.assign(dims, dims + rank);
    for (int64_t d : t.shape)
        if (d < 0) ICX_FAIL(ICX_ERR_SHAPE, "add_initializer: '%s' has a negative dimension", name);
    const size_t bytes = (size_t)numel(t.shape) * dtype_size(dtype);
    if (bytes && !host_data) ICX_FAIL(ICX_ERR_INVALID_ARG, "add_initializer: '%s' has no data", name);
    if (bytes) t.data.assign(static_cast<const uint8_t*>(host_data), static_cast<const uint8_t*>(host_data) + bytes);
    g->inits[name] = std::move(t);
    g->invalidate();
    return ICX_OK;
}

extern "C" int icx_graph_add_node(icx_graph* g, const char* name, const char* op_type, int n_in,
                                  const char* const* inputs, int n_out, const char* const* outputs,
                                  int n_attr, const char* const* attr_names,
                                  const int64_t* attr_values) {
    icx::clear_error();
    if (!g || !name || !op_type || n_in < 0 || n_out < 1 || !outputs || n_attr < 0 ||
        (n_attr && (!attr_names || !attr_values)))
        ICX_FAIL(ICX_ERR_INVALID_ARG, "add_node: bad arguments");
    if (g->find_node(name)) ICX_FAIL(ICX_ERR_INVALID_ARG, "add_node: a node named '%s' exists", name);
    Node n;
    n.name = name;
    n.op = op_type;
    n.in = names_of(n_in, inputs);
    n.out = names_of(n_out, outputs);
    for (int i = 0; i < n_attr; ++i) n.attr[attr_names[i] ? attr_names[i] : ""] = attr_values[i];
    g->nodes.push_back(std::move(n));
    g->invalidate();
    return ICX_OK;
}

extern "C" int icx_graph_set_node_attr_float(icx_graph* g, const char* node, const char* attr, double value) {
    icx::clear_error();
    if (!g || !node || !attr) ICX_FAIL(ICX_ERR_INVALID_ARG, "set_node_attr_float: bad arguments");
    Node* n = g->find_node(node);
    if (!n) ICX_FAIL(ICX_ERR_INVALID_ARG, "set_node_attr_float: no node '%s'", node);
    n->fattr[attr] = value;
    g->invalidate();
    return ICX_OK;
}

extern "C" int icx_graph_set_node_attr_ints(icx_graph* g, const char* node, const char* attr, int count,
                                            const int64_t* values) {
    icx::clear_error();
    if (!g || !node || !attr || count < 0 || (count && !values))
        ICX_FAIL(ICX_ERR_INVALID_ARG, "set_node_attr_ints: bad arguments");
    Node* n = g->find_node(node);
    if (!n) ICX_FAIL(ICX_ERR_INVALID_ARG, "set_node_attr_ints: no node '%s'", node);
    n->iattrs[attr] = std::vector<int64_t>(values, values + count);
    g->invalidate();
    return ICX_OK;
}

extern "C" int icx_graph_set_option(icx_graph* g, const char* name, int64_t value) {
    icx::clear_error();
    if (!g || !name) ICX_FAIL(ICX_ERR_INVALID_ARG, "set_option: bad arguments");
    bool* flag = nullptr;
    if (std::strcmp(name, "quantized_outputs") == 0) flag = &g->quant_out_on;
    if (std::strcmp(name, "quantized_inputs") == 0) flag = &g->qin_on;
    if (flag) {
        if (value != 0 && value != 1) ICX_FAIL(ICX_ERR_INVALID_ARG, "set_option: %s is 0 or 1", name);
        if (*flag != (value != 0)) {
            *flag = value != 0;
            g->invalidate();
        }
        return ICX_OK;
    }
    ICX_FAIL(ICX_ERR_INVALID_ARG, "set_option: no option '%s'", name);
}

extern "C" int icx_graph_add_output(icx_graph* g, const char* name) {
    icx::clear_error();
    if (!g || !name) ICX_FAIL(ICX_ERR_INVALID_ARG, "add_output: bad arguments");
    if (std::find(g->outputs.begin(), g->outputs.end(), name) == g->outputs.end()) {
        g->outputs.emplace_back(name);
        g->invalidate();
    }
    return ICX_OK;
}

static int icx_graph_plan_impl(icx_graph* g, char* buf, size_t buf_len) {
    if (!g) ICX_FAIL(ICX_ERR_INVALID_ARG, "plan: null graph");
    if (!g->planned) {
        Planner p(*g);
        const int rc = p.run();
        if (rc) return rc;
    }
    if (buf && buf_len) {
        std::ostringstream o;
        // execution order; each fused head is followed by the nodes folded into it
        for (auto& op : g->plan) {
            if (op.kind == Kind::Skip) continue;
            o << op.node.name << " " << op.node.op << " " << kind_name(op.kind) << " " << pattern_name(op.pattern);
            if (op.kind == Kind::FusedHead) {
                o << " steps=" << op.steps.size();
                if (op.w_zp_folded) o << " wzp=folded";
                if (!op.group.empty()) o << " group=" << op.group;
                o << " out=" << op.out;
            }
            o << "\n";
            for (auto& m : op.members)
                o << m.name << " " << m.op << " " << kind_name(Kind::Skip) << " " << pattern_name(op.pattern) << "\n";
        }
        for (auto& r : g->rowsum_wanted) o << "rowsum " << r << "\n";
        for (auto& r : g->range_wanted) o << "range " << r << "\n";
        for (auto& q : g->quant_out) o << "quantout " << q.first << " " << q.second.name << "\n";
        if (g->quant_fused) o << "quantout-launches " << g->quant_fused << "\n";
        for (auto& q : g->qin) o << "quantin " << q.first << " " << q.second.name << "\n";
        if (g->qin_fused) o << "quantin-launches " << g->qin_fused << "\n";
        if (g->dql_single) o << "dql-single-launches " << g->dql_single << "\n";
        const std::string s = o.str();
        if (s.size() + 1 > buf_len)
            ICX_FAIL(ICX_ERR_INVALID_ARG, "plan: summary needs %zu bytes, buffer has %zu", s.size() + 1, buf_len);
        std::memcpy(buf, s.c_str(), s.size() + 1);
    }
    return ICX_OK;
}

static int icx_graph_compile_impl(icx_graph* g, icx_stream_t stream) {
    if (!g) ICX_FAIL(ICX_ERR_INVALID_ARG, "compile: null graph");
    int rc = icx_graph_plan_impl(g, nullptr, 0);
    if (rc) return rc;
    if (g->compiled) return ICX_OK;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (g->ran && g->last_stream) ICX_HIP_CHECK(hipStreamSynchronize(g->last_stream));
    g->clear_run();
    g->free_weights();
    // the range-exchange buffer, for quantized-output GEMMs / attentions and single-launch DQLs
    bool exchange = !g->quant_out.empty();
    for (auto& op : g->plan)
        if (op.kind == Kind::Regular && op.node.op == "DynamicQuantizeLinear") exchange = true;
    if (exchange) {  // zeroed once; every launch leaves it valid for the next
        ICX_HIP_CHECK(hipMalloc(&g->qsync, icx::kQoutSyncBytes));
        ICX_HIP_CHECK(hipMemsetAsync(g->qsync, 0, icx::kQoutSyncBytes, s));
        ICX_HIP_CHECK(hipStreamSynchronize(s));
    }
    // initializers read as a MatMulInteger weight are packed once: B'^T [N,K] + colsum
    std::set<std::string> gemm_w;
    for (auto& op : g->plan) {
        if (op.kind == Kind::Skip) continue;
        if (op.pattern == Pattern::QuantizedLinear && op.group.empty()) gemm_w.insert(op.w);
        if (op.kind == Kind::Regular && op.node.op == "MatMulInteger" && op.node.in.size() > 1) {
            auto it = g->inits.find(op.node.in[1]);
            if (it != g->inits.end() && it->second.shape.size() == 2) gemm_w.insert(op.node.in[1]);
        }
    }
    for (auto& kv : g->inits) {
        const HostTensor& h = kv.second;
        DevTensor t;
        t.dtype = h.dtype;
        t.shape = h.shape;
        t.bytes = h.data.size();
        ICX_HIP_CHECK(hipMalloc(&t.ptr, std::max<size_t>(t.bytes, 4)));
        g->weights[kv.first] = t;
        if (t.bytes) ICX_HIP_CHECK(hipMemcpyAsync(t.ptr, h.data.data(), t.bytes, hipMemcpyHostToDevice, s));
        if (!gemm_w.count(kv.first)) continue;
        if (h.dtype != ICX_I8 && h.dtype != ICX_U8)
            ICX_FAIL(ICX_ERR_DTYPE, "MatMulInteger: b '%s' dtype %s unsupported (must be Int8 or UInt8)",
                     kv.first.c_str(), dtype_name(h.dtype));
        PackedW pw;
        pw.K = h.shape[0];
        pw.N = h.shape[1];
        pw.dtype = h.dtype;
        ICX_HIP_CHECK(hipMalloc(&pw.packed, std::max<size_t>(icx_packed_weight_bytes(pw.K, pw.N), 16)));
        ICX_HIP_CHECK(hipMalloc(&pw.colsum, std::max<size_t>(4 * (size_t)pw.N, 4)));
        g->packed[kv.first] = pw;
        if (pw.K && pw.N) {
            rc = icx_pack_weight(stream, t.ptr, h.dtype, pw.K, pw.N, pw.packed, pw.colsum);
            if (rc) return rc;
        }
    }
    // sibling groups: the column-concatenated weight, packed, and the concatenated column
    // operands of their chains
    for (auto& lead : g->plan) {
        if (lead.group_members.empty()) continue;
        std::vector<const PlannedOp*> hs;
        for (int k : lead.group_members) hs.push_back(&g->plan[k]);
        const HostTensor& w0 = g->inits.at(lead.w);
        const int64_t K = w0.shape[0], nh = w0.shape[1], n = (int64_t)hs.size();
        HostTensor cat;
        cat.dtype = w0.dtype;
        cat.shape = {K, n * nh};
        cat.data.resize((size_t)(K * n * nh));
        for (int64_t s_i = 0; s_i < n; ++s_i) {
            const HostTensor& w = g->inits.at(hs[s_i]->w);
            for (int64_t k = 0; k < K; ++k)
                std::memcpy(&cat.data[(size_t)(k * n * nh + s_i * nh)], &w.data[(size_t)(k * nh)], (size_t)nh);
        }
        int8_t* raw = nullptr;
        ICX_HIP_CHECK(hipMalloc(&raw, std::max<size_t>(cat.data.size(), 16)));
        DevTensor rt;
        rt.ptr = raw;
        rt.dtype = cat.dtype;
        rt.shape = cat.shape;
        rt.bytes = cat.data.size();
        g->weights[lead.group_w + ".raw"] = rt;
        ICX_HIP_CHECK(hipMemcpyAsync(raw, cat.data.data(), cat.data.size(), hipMemcpyHostToDevice, s));
        PackedW pw;
        pw.K = K;
        pw.N = n * nh;
        pw.dtype = cat.dtype;
        ICX_HIP_CHECK(hipMalloc(&pw.packed, std::max<size_t>(icx_packed_weight_bytes(pw.K, pw.N), 16)));
        ICX_HIP_CHECK(hipMalloc(&pw.colsum, std::max<size_t>(4 * (size_t)pw.N, 4)));
        g->packed[lead.group_w] = pw;
        rc = icx_pack_weight(stream, raw, cat.dtype, pw.K, pw.N, pw.packed, pw.colsum);
        if (rc) return rc;
        // the host copies must outlive the asynchronous uploads: synchronise per group
        std::vector<std::vector<float>> host_ops;
        for (size_t k = 0; k < lead.group_steps.size(); ++k) {
            for (int which = 0; which < 2; ++which) {
                const std::string& nm = which ? lead.group_steps[k].opnd1 : lead.group_steps[k].opnd0;
                if (nm.empty() || g->weights.count(nm) || g->inits.count(nm) ||
                    nm.compare(0, lead.out.size() + 2, lead.out + "::") != 0)
                    continue;
                std::vector<float> col((size_t)(n * nh));
                for (int64_t s_i = 0; s_i < n; ++s_i) {
                    const HostTensor& c = g->inits.at(which ? hs[s_i]->steps[k].opnd1 : hs[s_i]->steps[k].opnd0);
                    const float* src = reinterpret_cast<const float*>(c.data.data());
                    const bool sc = numel(c.shape) == 1;
                    for (int64_t j = 0; j < nh; ++j) col[(size_t)(s_i * nh + j)] = sc ? src[0] : src[j];
                }
                DevTensor t;
                t.dtype = ICX_F32;
                t.shape = {n * nh};
                t.bytes = col.size() * 4;
                ICX_HIP_CHECK(hipMalloc(&t.ptr, t.bytes));
                g->weights[nm] = t;
                ICX_HIP_CHECK(hipMemcpyAsync(t.ptr, col.data(), t.bytes, hipMemcpyHostToDevice, s));
                host_ops.push_back(std::move(col));
            }
        }
        ICX_HIP_CHECK(hipStreamSynchronize(s));
    }
    ICX_HIP_CHECK(hipStreamSynchronize(s));
    g->compiled = true;
    return ICX_OK;
}

extern "C" int icx_graph_set_input(icx_graph* g, const char* name, int dtype, int rank,
                                   const int64_t* dims, const void* data, int on_device) {
    icx::clear_error();
    if (!g || !name || rank < 0 || (rank && !dims)) ICX_FAIL(ICX_ERR_INVALID_ARG, "set_input: bad arguments");
    if (!valid_dtype(dtype) && dtype != ICX_I64)
        ICX_FAIL(ICX_ERR_DTYPE, "set_input: '%s' has unsupported dtype %d", name, dtype);
    BoundInput b;
    b.dtype = dtype;
    b.shape.assign(dims, dims + rank);
    for (int64_t d : b.shape)
        if (d < 0) ICX_FAIL(ICX_ERR_SHAPE, "set_input: '%s' has a negative dimension", name);
    const size_t bytes = (size_t)numel(b.shape) * dtype_size(dtype);
    if (bytes && !data) ICX_FAIL(ICX_ERR_INVALID_ARG, "set_input: '%s' has no data", name);
    if (g->hip_exec) {  // a captured run reads the bound device pointers in place
        auto old = g->bound.find(name);
        if (!on_device || old == g->bound.end() || old->second.dev != data || old->second.shape != b.shape ||
            old->second.dtype != dtype)
            g->drop_capture();
    }
    if (on_device) {
        b.dev = data;
    } else if (bytes) {
        // the last run may still be copying from the host buffer this one replaces
        auto old = g->bound.find(name);
        if (g->ran && g->last_stream && old != g->bound.end() && !old->second.dev)
            ICX_HIP_CHECK(hipStreamSynchronize(g->last_stream));
        b.host.assign(static_cast<const uint8_t*>(data), static_cast<const uint8_t*>(data) + bytes);
    }
    g->bound[name] = std::move(b);
    return ICX_OK;
}

// Per-op timing of one eager run (icx_graph_run_profiled): the reference's GpuEventTimer
// (src/cuda/inference/gpu_event_timer.rs:61-117) — an event after the input uploads, then one
// after each executed op, so op k's GPU time is the interval between events k and k + 1 —
// and the host time each op's validation and enqueue took (Executor::run_with_profiling,
// src/cuda/executor/variants.rs:415-515).
struct RunProfile {
    std::vector<std::pair<std::string, std::string>> ops;  // (label, node) per executed op
    std::vector<double> cpu_us;
};

// The reference's op_label (src/cuda/executor/variants.rs:35-56): a fused head is
// "Fused_<pattern>", any other op its type.
static std::string op_label(const PlannedOp& op) {
    return op.kind == Kind::FusedHead ? std::string("Fused_") + pattern_name(op.pattern) : op.node.op;
}

static int prof_event(icx_graph* g, size_t k, hipStream_t s) {
    while (g->prof_events.size() <= k) {
        // no system-scope fence: an ordinary event's cache write-back and invalidate would
        // add a few microseconds to every op it brackets; the run ends with a stream
        // synchronisation before anything is read
        hipEvent_t e;
        ICX_HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
        g->prof_events.push_back(e);
    }
    ICX_HIP_CHECK(hipEventRecord(g->prof_events[k], s));
    return ICX_OK;
}

static int icx_graph_run_impl(icx_graph* g, icx_stream_t stream, RunProfile* prof = nullptr) {
    if (!g) ICX_FAIL(ICX_ERR_INVALID_ARG, "run: null graph");
    int rc = icx_graph_compile_impl(g, stream);
    if (rc) return rc;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    // input shape guard (src/cuda/inference/mod.rs:441-460), before any GPU work
    for (auto& in : g->inputs) {
        auto b = g->bound.find(in.first);
        if (b == g->bound.end()) continue;
        const auto& want = in.second;
        const auto& got = b->second.shape;
        bool bad = want.size() != got.size();
        for (size_t i = 0; !bad && i < want.size(); ++i) bad = want[i] >= 0 && want[i] != got[i];
        if (bad)
            ICX_FAIL(ICX_ERR_SHAPE,
                     "input '%s' shape %s does not match the compiled plan's input dims %s (-1 = dynamic)",
                     in.first.c_str(), shape_str(got).c_str(), shape_str(want).c_str());
    }
    if (g->ran && g->last_stream && g->last_stream != s) ICX_HIP_CHECK(hipStreamSynchronize(g->last_stream));
    g->clear_run();
    g->last_stream = s;
    g->ran = true;
    Runner r(*g, s);
    if (prof && (rc = prof_event(g, 0, s))) return rc;
    rc = r.bind_inputs();
    if (rc) return rc;
    if (prof && (rc = prof_event(g, 1, s))) return rc;
    for (size_t i = 0; i < g->plan.size(); ++i) {
        const PlannedOp& op = g->plan[i];
        if (op.kind == Kind::Skip) continue;
        const auto t0 = std::chrono::steady_clock::now();
        rc = r.dispatch(op);
        if (rc) {
            const std::string msg = icx_last_error();
            set_error("node '%s' (%s): %s", op.node.name.c_str(), op.node.op.c_str(), msg.c_str());
            return rc;
        }
        if (prof) {
            prof->cpu_us.push_back(
                std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count());
            prof->ops.emplace_back(op_label(op), op.node.name);
            if ((rc = prof_event(g, prof->ops.size() + 1, s))) return rc;
        }
        r.release_dead(i);
    }
    return r.finish_outputs();
}

static int icx_graph_run_profiled_impl(icx_graph* g, icx_stream_t stream, icx_op_profile* ops, int capacity,
                                       int* n_ops, float* upload_us) {
    if (!g || !n_ops || capacity < 0 || (capacity && !ops))
        ICX_FAIL(ICX_ERR_INVALID_ARG, "run_profiled: bad arguments");
    *n_ops = 0;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    ICX_HIP_CHECK(hipStreamIsCapturing(reinterpret_cast<hipStream_t>(stream), &cap));
    if (cap != hipStreamCaptureStatusNone)
        ICX_FAIL(ICX_ERR_INVALID_ARG, "run_profiled: the stream is being captured (profile an eager run)");
    RunProfile prof;
    int rc = icx_graph_run_impl(g, stream, &prof);
    if (rc) return rc;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    ICX_HIP_CHECK(hipStreamSynchronize(s));  // one synchronisation for every event (finalize)
    float ms = 0.0f;
    if (upload_us) {
        ICX_HIP_CHECK(hipEventElapsedTime(&ms, g->prof_events[0], g->prof_events[1]));
        *upload_us = 1000.0f * ms;
    }
    const int n = (int)prof.ops.size();
    *n_ops = n;
    for (int k = 0; k < n && k < capacity; ++k) {
        icx_op_profile& o = ops[k];
        std::memset(&o, 0, sizeof o);
        std::snprintf(o.label, sizeof o.label, "%s", prof.ops[k].first.c_str());
        std::snprintf(o.node, sizeof o.node, "%s", prof.ops[k].second.c_str());
        ICX_HIP_CHECK(hipEventElapsedTime(&ms, g->prof_events[k + 1], g->prof_events[k + 2]));
        o.gpu_us = 1000.0f * ms;
        o.cpu_us = (float)prof.cpu_us[k];
    }
    return ICX_OK;
}

extern "C" int icx_graph_run_profiled(icx_graph* g, icx_stream_t stream, icx_op_profile* ops, int capacity,
                                      int* n_ops, float* upload_us) {
    icx::clear_error();
    try {
        return icx_graph_run_profiled_impl(g, stream, ops, capacity, n_ops, upload_us);
    } catch (const std::exception& e) {
        set_error("icx_graph_run_profiled: %s", e.what());
        return ICX_ERR_INVALID_ARG;
    }
}

// Capture: a warm-up run sizes the pool and the workspace, so that a second run reaches no
// hipMalloc, synchronisation or memset; that run is recorded into a HIP graph (nothing
// executes while recording) and instantiated.  Replay launches it; the outputs are then in
// the buffers the recording run assigned, which the replay restores as the graph's values.
static int icx_graph_capture_impl(icx_graph* g, icx_stream_t stream) {
    if (!g) ICX_FAIL(ICX_ERR_INVALID_ARG, "capture: null graph");
    for (auto& b : g->bound)
        if (!b.second.dev)
            ICX_FAIL(ICX_ERR_INVALID_ARG,
                     "capture: input '%s' is bound from host memory; a captured run reads its "
                     "inputs in place, so bind them on the device", b.first.c_str());
    if (!stream) ICX_FAIL(ICX_ERR_INVALID_ARG, "capture: the legacy default stream cannot be captured; pass a created stream");
    g->drop_capture();
    int rc = icx_graph_run_impl(g, stream);  // warm-up (executes)
    if (rc) return rc;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    ICX_HIP_CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed));
    rc = icx_graph_run_impl(g, stream);  // recorded
    hipGraph_t graph = nullptr;
    const hipError_t e = hipStreamEndCapture(s, &graph);
    if (rc) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc;
    }
    if (e != hipSuccess || !graph)
        ICX_FAIL(ICX_ERR_HIP, "capture: hipStreamEndCapture: %s", hipGetErrorString(e));
    hipGraphExec_t exec = nullptr;
    const hipError_t ie = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (ie != hipSuccess) {
        (void)hipGraphDestroy(graph);
        ICX_FAIL(ICX_ERR_HIP, "capture: hipGraphInstantiate: %s", hipGetErrorString(ie));
    }
    g->hip_graph = graph;
    g->hip_exec = exec;
    g->captured_values = g->values;
    return ICX_OK;
}

extern "C" int icx_graph_capture(icx_graph* g, icx_stream_t stream) {
    icx::clear_error();
    try {
        return icx_graph_capture_impl(g, stream);
    } catch (const std::exception& e) {
        set_error("icx_graph_capture: %s", e.what());
        return ICX_ERR_INVALID_ARG;
    }
}

extern "C" int icx_graph_replay(icx_graph* g, icx_stream_t stream) {
    icx::clear_error();
    if (!g) ICX_FAIL(ICX_ERR_INVALID_ARG, "replay: null graph");
    if (!g->hip_exec) ICX_FAIL(ICX_ERR_INVALID_ARG, "replay: nothing captured (call icx_graph_capture)");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (g->ran && g->last_stream && g->last_stream != s) ICX_HIP_CHECK(hipStreamSynchronize(g->last_stream));
    if (g->values.size() != g->captured_values.size() ||
        !std::equal(g->values.begin(), g->values.end(), g->captured_values.begin(),
                    [](const auto& a, const auto& b) { return a.first == b.first && a.second.ptr == b.second.ptr; })) {
        // an eager run since the capture moved the outputs: return its buffers to the pool
        // and restore the captured ones (they are the pool's free buffers the graph writes)
        g->clear_run();
        for (auto& kv : g->captured_values) {
            DevTensor t = kv.second;
            t.pooled = false;  // owned by the pool's free list, written by the graph
            g->values[kv.first] = t;
        }
    }
    ICX_HIP_CHECK(hipGraphLaunch(g->hip_exec, s));
    g->last_stream = s;
    g->ran = true;
    return ICX_OK;
}

extern "C" int icx_graph_status(icx_graph* g, icx_stream_t stream) {
    icx::clear_error();
    if (!g) ICX_FAIL(ICX_ERR_INVALID_ARG, "status: null graph");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    // the last run may have gone to another stream than the one given here: wait for it too
    if (g->ran && g->last_stream && g->last_stream != s) ICX_HIP_CHECK(hipStreamSynchronize(g->last_stream));
    if (!g->qsync) {
        ICX_HIP_CHECK(hipStreamSynchronize(s));
        return ICX_OK;
    }
    return icx::exchange_status(s, g->qsync);
}

extern "C" int icx_graph_get_output(icx_graph* g, const char* name, int* dtype, int* rank,
                                    int64_t* dims, const void** device_ptr) {
    icx::clear_error();
    if (!g || !name) ICX_FAIL(ICX_ERR_INVALID_ARG, "get_output: bad arguments");
    auto v = g->values.find(name);
    if (v == g->values.end()) ICX_FAIL(ICX_ERR_INVALID_ARG, "get_output: '%s' is not an output of the last run", name);
    const DevTensor& t = v->second;
    if (t.shape.size() > 8) ICX_FAIL(ICX_ERR_SHAPE, "get_output: '%s' has rank %zu > 8", name, t.shape.size());
    if (dtype) *dtype = t.dtype;
    if (rank) *rank = (int)t.shape.size();
    if (dims) std::copy(t.shape.begin(), t.shape.end(), dims);
    if (device_ptr) *device_ptr = t.ptr;
    return ICX_OK;
}

extern "C" int icx_graph_pool_stats(icx_graph* g, int64_t* hipmallocs, int64_t* hits,
                                    int64_t* bytes_held) {
    icx::clear_error();
    if (!g) ICX_FAIL(ICX_ERR_INVALID_ARG, "pool_stats: null graph");
    if (hipmallocs) *hipmallocs = g->pool.mallocs_;
    if (hits) *hits = g->pool.hits_;
    if (bytes_held) *bytes_held = g->pool.held_;
    return ICX_OK;
}

extern "C" int icx_graph_plan(icx_graph* g, char* buf, size_t buf_len) {
    icx::clear_error();
    try {
        return icx_graph_plan_impl(g, buf, buf_len);
    } catch (const std::exception& e) {
        set_error("icx_graph_plan: %s", e.what());
        return ICX_ERR_INVALID_ARG;
    }
}

extern "C" int icx_graph_compile(icx_graph* g, icx_stream_t stream) {
    icx::clear_error();
    try {
        return icx_graph_compile_impl(g, stream);
    } catch (const std::exception& e) {
        set_error("icx_graph_compile: %s", e.what());
        return ICX_ERR_INVALID_ARG;
    }
}

extern "C" int icx_graph_run(icx_graph* g, icx_stream_t stream) {
    icx::clear_error();
    try {
        return icx_graph_run_impl(g, stream);
    } catch (const std::exception& e) {
        set_error("icx_graph_run: %s", e.what());
        return ICX_ERR_INVALID_ARG;
    }
}
