// Graph executor for the quantized-linear path: the MI355X counterpart of the reference's
// GpuGraphExecutor shim (src/cuda/inference/mod.rs:208-659), its lowering (ir::lower,
// src/ir/lowering.rs:31-238) and per-op dispatch (src/cuda/executor/mod.rs:107-597).
//
//   build:   add_input / add_initializer / add_node / add_output (host only)
//   plan:    requested outputs (or the graph's sinks, mod.rs:505-519) and dead-node
//            elimination; topological sort; fusion decision: a QuantizedLinear head over
//            MatMulInteger -> Cast -> Mul -> [Add] -> [chain], elementwise chains reported
//            as MulAdd / AddMul / SubMul / DivMul when they are exactly those two ops;
//            weight zero-point folding; last use of every tensor            (host only)
//   compile: upload initializers, pack MatMulInteger weights once (icx_pack_weight)
//   run:     input shape guard, then every planned op on the caller's stream; intermediate
//            tensors come from a size-class pool on hipMalloc and return to it at their
//            last use (stream order makes the reuse safe).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <exception>
#include <map>
#include <set>
#include <sstream>
#include <string>
#include <vector>

#include "icx_common.hpp"

namespace {

using icx::set_error;

size_t dtype_size(int dt) { return (dt == ICX_I8 || dt == ICX_U8) ? 1 : 4; }

const char* dtype_name(int dt) {
    switch (dt) {
        case ICX_I8: return "Int8";
        case ICX_U8: return "UInt8";
        case ICX_I32: return "Int32";
        case ICX_F32: return "Float32";
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
    int64_t attr_or(const std::string& k, int64_t d) const {
        auto it = attr.find(k);
        return it == attr.end() ? d : it->second;
    }
};

// One step of an elementwise chain: v = v op operand (or operand op v).  The operand is a
// tensor, or the product of two (a folded Mul(x_scale, w_scale) node).
struct Step {
    int op = ICX_OP_MUL;
    bool lhs = false;
    std::string opnd0, opnd1;
};

enum class Kind { Regular, FusedHead, Skip };
enum class Pattern { None, QuantizedLinear, MulAdd, AddMul, SubMul, DivMul, ElementwiseChain };

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
        default: return "-";
    }
}

// One entry of the execution plan (the reference's PlannedOp, src/ir/plan.rs).
struct PlannedOp {
    Node node;
    Kind kind = Kind::Regular;
    Pattern pattern = Pattern::None;
    std::string a, w, a_zp, w_zp;  // QuantizedLinear: the MatMulInteger operands
    bool w_zp_folded = false;      // all-zero weight zero point dropped
    std::string chain_in, out;     // chain input (elementwise heads) and fused output
    std::vector<Step> steps;
    std::vector<std::pair<std::string, std::string>> members;  // (name, op) folded in
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
    std::vector<PlannedOp> plan;
    std::vector<std::string> live_outputs;   // requested outputs, or the sinks
    std::map<std::string, size_t> last_use;  // tensor -> plan index of its last reader
    std::set<std::string> rowsum_wanted;     // DQL outputs whose row sums a GEMM reads

    // device state
    std::map<std::string, DevTensor> weights;      // uploaded initializers
    std::map<std::string, PackedW> packed;         // packed MatMulInteger weights
    std::map<std::string, BoundInput> bound;       // inputs for the next run
    std::map<std::string, DevTensor> values;       // tensors of the current / last run
    std::map<std::string, std::string> rowsum_of;  // DQL y -> its row-sum tensor
    hipStream_t last_stream = nullptr;
    bool ran = false;
    Pool pool;
    void* ws = nullptr;
    size_t ws_bytes = 0;

    ~icx_graph() {
        if (ran && last_stream) (void)hipStreamSynchronize(last_stream);
        clear_run();
        free_weights();
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
    }
    void clear_run() {
        for (auto& kv : values)
            if (kv.second.pooled) pool.put(kv.second.ptr, kv.second.cls);
        values.clear();
        rowsum_of.clear();
    }
    void invalidate() { planned = compiled = false; }
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
        gi_ = GraphIndex(nodes_);
        outs_.clear();
        outs_.insert(g_.live_outputs.begin(), g_.live_outputs.end());
        const int n = (int)nodes_.size();
        std::vector<PlannedOp> ops(n);
        for (int i = 0; i < n; ++i) ops[i].node = nodes_[i];
        // quantized-linear heads first: they own their Cast / Mul / Add / chain nodes
        for (int pass = 0; pass < 2; ++pass) {
            for (int i = 0; i < n; ++i) {
                if (claimed_.count(i)) continue;
                PlannedOp head;
                head.node = nodes_[i];
                std::vector<int> mem;
                const bool hit = pass == 0 ? match_qlinear(i, head, mem) : match_chain(i, head, mem);
                if (!hit) continue;
                // The head runs at its last member's position: every operand of every member
                // is produced before that point, and nothing else reads the members' outputs.
                int pos = i;
                claimed_.insert(i);
                for (int m : mem) {
                    claimed_.insert(m);
                    pos = std::max(pos, m);
                    head.members.emplace_back(nodes_[m].name, nodes_[m].op);
                    ops[m].kind = Kind::Skip;
                }
                ops[i].kind = Kind::Skip;
                ops[pos] = head;
            }
        }
        g_.plan = ops;
        g_.rowsum_wanted.clear();
        for (auto& op : g_.plan) {
            if (op.pattern != Pattern::QuantizedLinear) continue;
            const bool u8w = g_.inits[op.w].dtype == ICX_U8;
            if (!u8w && (op.w_zp.empty() || op.w_zp_folded)) continue;
            auto p = gi_.producer.find(op.a);
            if (p != gi_.producer.end() && nodes_[p->second].op == "DynamicQuantizeLinear")
                g_.rowsum_wanted.insert(op.a);
        }
        g_.last_use.clear();
        for (size_t i = 0; i < g_.plan.size(); ++i) {
            const PlannedOp& op = g_.plan[i];
            if (op.kind == Kind::Skip) continue;
            std::vector<std::string> uses = op.node.in;
            for (auto& st : op.steps) {
                uses.push_back(st.opnd0);
                if (!st.opnd1.empty()) uses.push_back(st.opnd1);
            }
            if (!op.chain_in.empty()) uses.push_back(op.chain_in);
            for (auto& u : uses)
                if (!u.empty()) g_.last_use[u] = i;
        }
        g_.planned = true;
        return ICX_OK;
    }

   private:
    icx_graph& g_;
    GraphIndex gi_;
    std::vector<Node> nodes_;
    std::set<std::string> outs_;
    std::set<int> claimed_;

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
    // The single reader of t, or -1 (also when t is a live output: it must materialise).
    int sole_consumer(const std::string& t) const {
        if (outs_.count(t)) return -1;
        auto it = gi_.consumers.find(t);
        if (it == gi_.consumers.end() || it->second.size() != 1) return -1;
        return it->second[0];
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
    void extend_chain(std::string& cur, std::vector<Step>& steps, std::vector<int>& mem) const {
        while ((int)steps.size() < ICX_MAX_CHAIN) {
            const int c = sole_consumer(cur);
            Step st;
            if (c < 0 || !as_step(c, cur, st)) break;
            steps.push_back(st);
            mem.push_back(c);
            cur = nodes_[c].out[0];
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
        if (ci < 0 || nodes_[ci].op != "Cast" || nodes_[ci].attr_or("to", -1) != 1 || nodes_[ci].out.size() != 1)
            return false;
        const std::string cast_out = nodes_[ci].out[0];
        const int si = sole_consumer(cast_out);
        if (si < 0 || nodes_[si].op != "Mul" || nodes_[si].in.size() != 2 || nodes_[si].out.size() != 1) return false;
        const Node& s1 = nodes_[si];
        const bool left = s1.in[0] == cast_out, right = s1.in[1] == cast_out;
        if (left == right) return false;
        const std::string scale = left ? s1.in[1] : s1.in[0];
        Step st;
        st.op = ICX_OP_MUL;
        st.lhs = !left;
        mem = {ci, si};
        // scale = Mul(x_scale, w_scale) read only here: a product operand, rounded once
        auto sp = gi_.producer.find(scale);
        if (sp != gi_.producer.end() && nodes_[sp->second].op == "Mul" && nodes_[sp->second].in.size() == 2 &&
            sole_consumer(scale) == si && !claimed_.count(sp->second)) {
            st.opnd0 = nodes_[sp->second].in[0];
            st.opnd1 = nodes_[sp->second].in[1];
            mem.push_back(sp->second);
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

    // Two or more binary ops over one running tensor with static operands.
    bool match_chain(int ni, PlannedOp& head, std::vector<int>& mem) {
        const Node& n = nodes_[ni];
        if (op_code(n.op) < 0 || n.in.size() != 2 || n.out.size() != 1) return false;
        std::string in;
        if (static_f32(n.in[1]) && !static_f32(n.in[0])) in = n.in[0];
        else if (static_f32(n.in[0]) && !static_f32(n.in[1])) in = n.in[1];
        else return false;
        Step st;
        if (!as_step(ni, in, st)) return false;
        std::vector<Step> steps = {st};
        std::string cur = n.out[0];
        mem.clear();
        extend_chain(cur, steps, mem);
        if (steps.size() < 2) return false;
        head.kind = Kind::FusedHead;
        head.pattern = Pattern::ElementwiseChain;
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
            if (op.pattern == Pattern::QuantizedLinear) return run_qlinear(op);
            return run_chain(op.chain_in, op.steps, op.out, pattern_name(op.pattern));
        }
        const std::string& t = op.node.op;
        if (t == "DynamicQuantizeLinear") return run_dql(op.node);
        if (t == "MatMulInteger") return run_matmul_integer(op.node);
        if (t == "DequantizeLinear") return run_dequantize(op.node);
        if (t == "Cast") return run_cast(op.node);
        if (op_code(t) >= 0) return run_binary(op.node);
        set_error("op '%s' is not on the quantized-linear path", t.c_str());
        return ICX_ERR_UNSUPPORTED;
    }

    // Return to the pool every pooled tensor whose last reader was plan entry i, or that
    // nothing reads.  Live outputs stay until the next run.
    void release_dead(size_t i) {
        for (auto it = g_.values.begin(); it != g_.values.end();) {
            const std::string& name = it->first;
            const bool is_out =
                std::find(g_.live_outputs.begin(), g_.live_outputs.end(), name) != g_.live_outputs.end();
            std::string key = name;
            const size_t sfx = name.rfind("::rowsum");
            if (sfx != std::string::npos) key = name.substr(0, sfx);
            auto lu = g_.last_use.find(key);
            const bool dead = lu == g_.last_use.end() || lu->second <= i;
            if (it->second.pooled && !is_out && dead) {
                g_.pool.put(it->second.ptr, it->second.cls);
                it = g_.values.erase(it);
            } else {
                ++it;
            }
        }
    }

   private:
    icx_graph& g_;
    hipStream_t s_;

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
        set_error("%s: input tensor '%s' is missing", who, name.c_str());
        return ICX_ERR_INVALID_ARG;
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

    int chain_operand(const std::string& name, const std::vector<int64_t>& out_shape, const char* who,
                      int32_t* kind, const float** p) const {
        const DevTensor* t;
        int rc = need(name, &t, who);
        if (rc) return rc;
        if (t->dtype != ICX_F32) {
            set_error("%s: operand '%s' must be Float32, got %s", who, name.c_str(), dtype_name(t->dtype));
            return ICX_ERR_DTYPE;
        }
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

    int run_qlinear(const PlannedOp& op) {
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
        DevTensor* Y;
        rc = alloc(op.out, ICX_F32, oshape, &Y);
        if (rc) return rc;
        rc = workspace(icx_matmul_integer_workspace_size(M, pw.K, pw.N, 1));
        if (rc) return rc;
        return icx_qlinear_f32(s_, a_ptr, a_dt, pw.packed, pw.dtype, 1, pw.colsum, M, pw.K, pw.N, azp, bzp, blen,
                               rowsum, &ch, static_cast<float*>(Y->ptr), g_.ws, g_.ws_bytes);
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

    int run_dql(const Node& n) {
        if (n.in.size() != 1 || n.out.size() != 3) {
            set_error("DynamicQuantizeLinear: expected 1 input and 3 outputs, got %zu and %zu", n.in.size(),
                      n.out.size());
            return ICX_ERR_INVALID_ARG;
        }
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
        rc = workspace(icx_dql_workspace_size(cnt));
        if (rc) return rc;
        return icx_dynamic_quantize_linear(s_, x, cnt, static_cast<uint8_t*>(Y->ptr), static_cast<float*>(S->ptr),
                                           static_cast<uint8_t*>(Z->ptr), R ? static_cast<int32_t*>(R->ptr) : nullptr,
                                           row_len, g_.ws, g_.ws_bytes);
    }

    int run_chain(const std::string& in_name, const std::vector<Step>& steps, const std::string& out_name,
                  const char* who) {
        const DevTensor* X;
        int rc = need(in_name, &X, who);
        if (rc) return rc;
        if (X->dtype != ICX_F32) {
            set_error("%s: input '%s' must be Float32, got %s", who, in_name.c_str(), dtype_name(X->dtype));
            return ICX_ERR_DTYPE;
        }
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

    // Mul / Add / Sub / Div outside a chain: the output must have one operand's shape.
    int run_binary(const Node& n) {
        if (n.in.size() != 2 || n.out.size() != 1) {
            set_error("%s: expected 2 inputs and 1 output", n.op.c_str());
            return ICX_ERR_INVALID_ARG;
        }
        const DevTensor *A, *B;
        int rc = need(n.in[0], &A, n.op.c_str());
        if (!rc) rc = need(n.in[1], &B, n.op.c_str());
        if (rc) return rc;
        bool ok;
        const std::vector<int64_t> out = broadcast_shape(A->shape, B->shape, &ok);
        if (!ok) {
            set_error("%s: shapes %s and %s do not broadcast", n.op.c_str(), shape_str(A->shape).c_str(),
                      shape_str(B->shape).c_str());
            return ICX_ERR_SHAPE;
        }
        Step st;
        st.op = op_code(n.op);
        if (A->shape == out) {
            st.opnd0 = n.in[1];
            return run_chain(n.in[0], {st}, n.out[0], n.op.c_str());
        }
        if (B->shape == out) {
            st.lhs = true;
            st.opnd0 = n.in[0];
            return run_chain(n.in[1], {st}, n.out[0], n.op.c_str());
        }
        set_error("%s: broadcast of %s and %s to a new shape %s is not on this path", n.op.c_str(),
                  shape_str(A->shape).c_str(), shape_str(B->shape).c_str(), shape_str(out).c_str());
        return ICX_ERR_UNSUPPORTED;
    }

    int run_cast(const Node& n) {
        const DevTensor* X;
        int rc = need(n.in[0], &X, "Cast");
        if (rc) return rc;
        if (n.attr_or("to", -1) != 1) {
            set_error("Cast to ONNX dtype %lld is not on this path (FLOAT only)", (long long)n.attr_or("to", -1));
            return ICX_ERR_UNSUPPORTED;
        }
        if (X->dtype != ICX_I32 && X->dtype != ICX_F32) {
            set_error("Cast from %s to Float32 is not on this path", dtype_name(X->dtype));
            return ICX_ERR_UNSUPPORTED;
        }
        const std::vector<int64_t> shape = X->shape;
        const void* x = X->ptr;
        const int dt = X->dtype;
        const size_t cnt = (size_t)numel(shape);
        DevTensor* Y;
        rc = alloc(n.out[0], ICX_F32, shape, &Y);
        if (rc) return rc;
        if (dt == ICX_F32) {
            if (cnt) ICX_HIP_CHECK(hipMemcpyAsync(Y->ptr, x, cnt * 4, hipMemcpyDeviceToDevice, s_));
            return ICX_OK;
        }
        return icx_cast_i32_f32(s_, static_cast<const int32_t*>(x), cnt, static_cast<float*>(Y->ptr));
    }

    // DequantizeLinear (src/operators/dequantize_linear.rs:32-180): per-tensor or per-axis.
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
};

std::vector<std::string> names_of(int n, const char* const* p) {
    std::vector<std::string> v;
    for (int i = 0; i < n; ++i) v.emplace_back(p && p[i] ? p[i] : "");
    return v;
}

bool valid_dtype(int dt) { return dt == ICX_I8 || dt == ICX_U8 || dt == ICX_I32 || dt == ICX_F32; }

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
    if (!valid_dtype(dtype)) ICX_FAIL(ICX_ERR_DTYPE, "add_initializer: '%s' has unsupported dtype %d", name, dtype);
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
    icx::clear_error();
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
                o << " out=" << op.out;
            }
            o << "\n";
            for (auto& m : op.members)
                o << m.first << " " << m.second << " " << kind_name(Kind::Skip) << " " << pattern_name(op.pattern) << "\n";
        }
        for (auto& r : g->rowsum_wanted) o << "rowsum " << r << "\n";
        const std::string s = o.str();
        if (s.size() + 1 > buf_len)
            ICX_FAIL(ICX_ERR_INVALID_ARG, "plan: summary needs %zu bytes, buffer has %zu", s.size() + 1, buf_len);
        std::memcpy(buf, s.c_str(), s.size() + 1);
    }
    return ICX_OK;
}

static int icx_graph_compile_impl(icx_graph* g, icx_stream_t stream) {
    icx::clear_error();
    if (!g) ICX_FAIL(ICX_ERR_INVALID_ARG, "compile: null graph");
    int rc = icx_graph_plan_impl(g, nullptr, 0);
    if (rc) return rc;
    if (g->compiled) return ICX_OK;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (g->ran && g->last_stream) ICX_HIP_CHECK(hipStreamSynchronize(g->last_stream));
    g->clear_run();
    g->free_weights();
    // initializers read as a MatMulInteger weight are packed once: B'^T [N,K] + colsum
    std::set<std::string> gemm_w;
    for (auto& op : g->plan) {
        if (op.kind == Kind::Skip) continue;
        if (op.pattern == Pattern::QuantizedLinear) gemm_w.insert(op.w);
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
    ICX_HIP_CHECK(hipStreamSynchronize(s));
    g->compiled = true;
    return ICX_OK;
}

extern "C" int icx_graph_set_input(icx_graph* g, const char* name, int dtype, int rank,
                                   const int64_t* dims, const void* data, int on_device) {
    icx::clear_error();
    if (!g || !name || rank < 0 || (rank && !dims)) ICX_FAIL(ICX_ERR_INVALID_ARG, "set_input: bad arguments");
    if (!valid_dtype(dtype)) ICX_FAIL(ICX_ERR_DTYPE, "set_input: '%s' has unsupported dtype %d", name, dtype);
    BoundInput b;
    b.dtype = dtype;
    b.shape.assign(dims, dims + rank);
    for (int64_t d : b.shape)
        if (d < 0) ICX_FAIL(ICX_ERR_SHAPE, "set_input: '%s' has a negative dimension", name);
    const size_t bytes = (size_t)numel(b.shape) * dtype_size(dtype);
    if (bytes && !data) ICX_FAIL(ICX_ERR_INVALID_ARG, "set_input: '%s' has no data", name);
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

static int icx_graph_run_impl(icx_graph* g, icx_stream_t stream) {
    icx::clear_error();
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
    rc = r.bind_inputs();
    if (rc) return rc;
    for (size_t i = 0; i < g->plan.size(); ++i) {
        const PlannedOp& op = g->plan[i];
        if (op.kind == Kind::Skip) continue;
        rc = r.dispatch(op);
        if (rc) {
            const std::string msg = icx_last_error();
            set_error("node '%s' (%s): %s", op.node.name.c_str(), op.node.op.c_str(), msg.c_str());
            return rc;
        }
        r.release_dead(i);
    }
    return ICX_OK;
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
    try {
        return icx_graph_plan_impl(g, buf, buf_len);
    } catch (const std::exception& e) {
        set_error("icx_graph_plan: %s", e.what());
        return ICX_ERR_INVALID_ARG;
    }
}

extern "C" int icx_graph_compile(icx_graph* g, icx_stream_t stream) {
    try {
        return icx_graph_compile_impl(g, stream);
    } catch (const std::exception& e) {
        set_error("icx_graph_compile: %s", e.what());
        return ICX_ERR_INVALID_ARG;
    }
}

extern "C" int icx_graph_run(icx_graph* g, icx_stream_t stream) {
    try {
        return icx_graph_run_impl(g, stream);
    } catch (const std::exception& e) {
        set_error("icx_graph_run: %s", e.what());
        return ICX_ERR_INVALID_ARG;
    }
}
