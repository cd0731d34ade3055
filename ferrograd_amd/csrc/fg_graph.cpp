// fg_graph.cpp -- graph IR, lowering / fusion planner and plan executor.
//
// Replaces, behind the C ABI, the reference's graph compiler and runtime
// for the fused training path:
//   * graph IR and SaveIndicators: crates/fused_gpu/src/dispatch/backend/
//     mod.rs:499-1316 (Node, GraphOp, validate, compute_saved_nodes);
//   * lowering: kernel/{forward,backward,loss,optim}.rs driven by
//     kernel/mod.rs:107-152 -- which emits one generated kernel per root and
//     re-inlines elementwise chains into every consumer;
//   * buffers and scheduling: dispatch/mod.rs:509-845 and the hipGraph
//     capture of rocm/mod.rs:268-389.
//
// Lowering here pattern-matches the graph onto the hand-written gfx950
// kernels instead of generating code:
//   * matmul [-> bias add] [-> relu|gelu] becomes ONE GEMM launch whose
//     epilogue adds the bias, applies the activation and also stores the
//     pre-activation (kept for backward);
//   * runs of elementwise nodes of one shape become ONE elementwise-program
//     launch (fg_eltwise.h) that reads each external input once and writes
//     every node value;
//   * softmax followed by the CE loss becomes ONE fused softmax+CE launch
//     writing dlogits = p - onehot directly;
//   * backward is planned statically in reverse node order; the activation
//     derivative of a layer is fused into the epilogue of the dA GEMM of the
//     layer above (dZ_prev = (dZ W^T) * act'(Z_prev)), bias gradients are
//     column reductions, and every optimiser update is one multi-tensor
//     launch.
// All plan-owned tensors live in one 256-byte-aligned device arena.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <initializer_list>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <vector>

#include "fg_eltwise.h"
#include "fg_internal.h"

namespace {

constexpr int kNone = -1;

bool is_unary(int op) {
    switch (op) {
        case FG_OP_RELU: case FG_OP_GELU: case FG_OP_ELU: case FG_OP_TANH:
        case FG_OP_EXP: case FG_OP_LOG: case FG_OP_ABS: case FG_OP_NEG:
            return true;
        default:
            return false;
    }
}
bool is_binary_elt(int op) {
    return op == FG_OP_ADD || op == FG_OP_SUB || op == FG_OP_MUL || op == FG_OP_DIV ||
           op == FG_OP_BIAS_ADD;
}
bool is_elementwise(int op) { return is_unary(op) || is_binary_elt(op); }
int arity(int op) {
    if (op == FG_OP_INPUT || op == FG_OP_CONST) return 0;
    if (is_unary(op) || op == FG_OP_SOFTMAX) return 1;
    return 2;
}

const char *op_name(int op) {
    static const char *names[] = {"input", "const", "add",  "sub", "mul",  "div",
                                  "matmul", "relu", "gelu", "elu", "tanh", "exp",
                                  "log",   "abs",   "neg",  "softmax", "bias_add"};
    return (op >= 0 && op <= FG_OP_BIAS_ADD) ? names[op] : "?";
}

// SaveIndicator flags (kernel/mod.rs:41-93).
constexpr uint32_t kDefFwd = 1u, kDefBwd = 2u;

struct GNode {
    int op = FG_OP_INPUT;
    std::vector<uint32_t> in;
    std::vector<uint32_t> fields;  // Input: meta field per dim
    float value = 0.0f;            // Const (already rounded to dtype)
    uint32_t flags = 0;            // Input flags
    int dtype = FG_DTYPE_F32;      // Input / Const: declared; operations: of their first input
};

int esize(int dt) { return dt == FG_DTYPE_F32 ? 4 : 2; }
const char *dtype_name(int dt) {
    return dt == FG_DTYPE_F16 ? "f16" : dt == FG_DTYPE_BF16 ? "bf16" : "f32";
}

// Host rounding of an fp32 value to a 16-bit type and back (graph constants
// of F16 / BF16 type hold values of that type): nearest, ties to even.
float round_host(int dt, float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    if (dt == FG_DTYPE_BF16) {
        if ((u & 0x7fffffffu) <= 0x7f800000u) u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
    } else if (dt == FG_DTYPE_F16) {
        const float a = std::fabs(x);
        if (!(a < 65520.0f)) return a == a ? std::copysign(INFINITY, x) : x;
        // Scale so the f16 unit in the last place becomes an integer step of
        // the fp32 value, round with nearbyint (ties to even), scale back.
        int e;
        std::frexp(a, &e);
        const int ulp_exp = std::max(e - 11, -24);  // f16: 11-bit significand, min 2^-24
        const float r = std::ldexp(std::nearbyint(std::ldexp(x, -ulp_exp)), ulp_exp);
        std::memcpy(&u, &r, 4);
    }
    float r;
    std::memcpy(&r, &u, 4);
    return r;
}

struct Shape {
    bool scalar = false;
    bool vector = false;  // rank 1
    int64_t rows = 1, cols = 1;
    int64_t numel() const { return scalar ? 1 : rows * cols; }
};

}  // namespace

struct fg_graph {
    int loss = FG_LOSS_MSE;
    int optim = FG_OPTIM_SGD;
    uint32_t nfields = 0;
    std::vector<GNode> nodes;
};

namespace {

// --------------------------------------------------------- shape checks
int infer_shapes(const fg_graph &g, const uint32_t *meta, int n_meta, std::vector<Shape> &sh) {
    const size_t n = g.nodes.size();
    FG_REQUIRE(n > 0, FG_ERR_GRAPH, "graph has no nodes");
    FG_REQUIRE(n_meta >= (int)g.nfields + 1, FG_ERR_GRAPH,
               "metadata has %d fields, graph declares %u dims (+1 for lr)", n_meta, g.nfields);
    sh.assign(n, Shape{});
    for (size_t i = 0; i < n; ++i) {
        const GNode &nd = g.nodes[i];
        Shape s;
        switch (nd.op) {
            case FG_OP_INPUT: {
                FG_REQUIRE(!nd.fields.empty(), FG_ERR_GRAPH, "input %zu has rank 0", i);
                int64_t rows = 1;
                for (size_t d = 0; d < nd.fields.size(); ++d) {
                    const uint32_t f = nd.fields[d];
                    FG_REQUIRE(f >= 1 && f < (uint32_t)n_meta, FG_ERR_GRAPH,
                               "input %zu: missing metadata field %u", i, f);
                    FG_REQUIRE(meta[f] > 0, FG_ERR_SHAPE, "input %zu: dim %zu is 0", i, d);
                    if (d + 1 < nd.fields.size()) rows *= meta[f];
                }
                s.rows = rows;
                s.cols = meta[nd.fields.back()];
                s.vector = nd.fields.size() == 1;
                break;
            }
            case FG_OP_CONST:
                s.scalar = true;
                break;
            case FG_OP_MATMUL: {
                const Shape &a = sh[nd.in[0]], &b = sh[nd.in[1]];
                FG_REQUIRE(!a.scalar && !b.scalar && !a.vector && !b.vector, FG_ERR_SHAPE,
                           "matmul %zu: operands must be matrices", i);
                FG_REQUIRE(a.cols == b.rows, FG_ERR_SHAPE,
                           "matmul %zu: inner dims differ (%lld vs %lld)", i,
                           (long long)a.cols, (long long)b.rows);
                s.rows = a.rows;
                s.cols = b.cols;
                break;
            }
            case FG_OP_SOFTMAX: {
                const Shape &a = sh[nd.in[0]];
                FG_REQUIRE(!a.scalar, FG_ERR_SHAPE, "softmax %zu of a scalar", i);
                s = a;
                break;
            }
            default: {
                if (is_unary(nd.op)) {
                    FG_REQUIRE(!sh[nd.in[0]].scalar, FG_ERR_SHAPE, "%s %zu of a scalar",
                               op_name(nd.op), i);
                    s = sh[nd.in[0]];
                    break;
                }
                const Shape &a = sh[nd.in[0]], &b = sh[nd.in[1]];
                FG_REQUIRE(!(a.scalar && b.scalar), FG_ERR_SHAPE,
                           "%s %zu: both operands are constants", op_name(nd.op), i);
                if (nd.op == FG_OP_BIAS_ADD) {
                    FG_REQUIRE(!a.scalar && b.vector && b.cols == a.cols, FG_ERR_SHAPE,
                               "bias_add %zu: needs x[..., N] + b[N]", i);
                    s = a;
                } else if (a.scalar) {
                    s = b;
                } else if (b.scalar) {
                    s = a;
                } else if (a.rows == b.rows && a.cols == b.cols && a.vector == b.vector) {
                    s = a;
                } else if (b.vector && b.cols == a.cols) {
                    s = a;  // row broadcast of b
                } else if (a.vector && a.cols == b.cols) {
                    s = b;  // row broadcast of a
                } else {
                    fg::set_error("%s %zu: shapes [%lld,%lld] and [%lld,%lld] do not match",
                                  op_name(nd.op), i, (long long)a.rows, (long long)a.cols,
                                  (long long)b.rows, (long long)b.cols);
                    return FG_ERR_SHAPE;
                }
            }
        }
        sh[i] = s;
    }
    const int last_op = g.nodes.back().op;
    FG_REQUIRE(last_op != FG_OP_INPUT && last_op != FG_OP_CONST, FG_ERR_GRAPH,
               "the last node must be an operation");
    return FG_OK;
}

// ---------------------------------------------------------------- plan
enum LaunchKind {
    LK_GEMM,
    LK_GEMM_BWD,
    LK_BIAS_GRAD,
    LK_SOFTMAX,
    LK_SOFTMAX_BWD,
    LK_ELT,
    LK_SMCE,
    LK_FILL0,
};

struct Launch {
    int kind = LK_GEMM;
    int dtype = FG_DTYPE_F32;  // element type of the launch's tensors
    int layout = FG_NN, M = 0, N = 0, K = 0, lda = 0, ldb = 0, ldc = 0, ldz = 0;
    int act = FG_ACT_NONE, accumulate = 0;
    int accumulate2 = 0;  // TN GEMM with fused bias gradient: accumulate into sExtra
    int sA = kNone, sB = kNone, sC = kNone, sZ = kNone, sBias = kNone, sExtra = kNone;
    fg::EltProgram prog{};
    int src_slot[fg::kEltMaxSrc];
    int dst_slot[fg::kEltMaxDst];
    int label_slot = kNone;
    uint64_t count = 0;
    // The final forward softmax when the fused CE loss follows it: a captured
    // step leaves it out and the loss launch writes its output (sProbs).
    bool elidable = false;
    int sProbs = kNone;
    // A weight-gradient GEMM (fp32, TN) followed by the data-gradient GEMM
    // of the same layer (NT): the two read the same dZ and write different
    // gradients, so they go to fg::gemm_dw_dx_f32 together, which puts them
    // in one launch when both take small kernels.
    bool pair_next = false;
    // A forward GEMM (fp32, NN) whose output is the A operand of the next
    // launch, a forward GEMM (fp32, NN): the two go to
    // fg::gemm_fwd_chain_f32, where the second sums the first's K slices
    // when the first splits K and the second takes the skinny kernel.
    bool chain_next = false;
    std::string desc;
    Launch() {
        std::fill(src_slot, src_slot + fg::kEltMaxSrc, kNone);
        std::fill(dst_slot, dst_slot + fg::kEltMaxDst, kNone);
    }
};

struct Slot {
    uint64_t offset = 0;
    uint64_t bytes = 0;        // allocated (whole words)
    uint64_t used = 0;         // elements x element size
    bool external = false;
    void *ext = nullptr;
    int dtype = FG_DTYPE_F32;  // element type (u32 labels count as 4-byte elements)
};

struct Group {
    int mm = kNone, bias_node = kNone, bias_src = kNone, act_node = kNone;
    int pre = kNone;  // node holding the pre-activation value
    int fin = kNone;  // last node of the group
};

}  // namespace

struct fg_plan {
    fg_ctx *ctx = nullptr;
    fg_graph g;
    std::vector<uint32_t> meta;
    std::vector<Shape> shape;
    std::vector<std::vector<uint32_t>> users;
    std::vector<uint32_t> save;
    std::vector<char> needs_grad;
    std::vector<int> val_slot, grad_slot, group_of;
    std::vector<Group> groups;
    std::vector<Slot> slots;
    char *arena = nullptr;
    uint64_t arena_bytes = 0;
    std::vector<int> dtype;        // element type per node
    std::vector<uint32_t> inputs;  // input node ids in order
    std::vector<int> input_slot;
    int target_slot = kNone, loss_slot = kNone, mean_slot = kNone, adam_slot = kNone;
    uint64_t target_bytes = 0;
    int last = 0;
    bool ce_fused_possible = false;
    bool ce_fused_pending = false;
    std::vector<Launch> fwd, loss, bwd_seed, bwd_fused;
    std::vector<int> m_slot, v_slot;
    std::vector<uint32_t> opt_inputs;  // indices into inputs that the optimiser updates
    fg_mt *mt_all = nullptr;
    std::vector<fg_mt *> mt_single;
    // Captured Adam steps update the optimised inputs in groups, each on a
    // second stream as soon as the backward is done with its tensors:
    // mt_group_after[g] is the index (in the captured backward list) of the
    // last launch of the launch group after which nothing in the backward
    // touches group g's parameters or gradients (-1: nothing does).
    std::vector<fg_mt *> mt_groups;
    std::vector<int> mt_group_after;
    hipStream_t side = nullptr;        // that second stream (default priority)
    std::vector<hipEvent_t> events;    // one per group, then the join, then the fork
    bool hold_mean = false;            // capture: the loss leaves its mean to the side stream
    bool mt_dirty = true;
    float lr = 1e-3f, b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
    // The plan's own view of its context: same device and stream, with a
    // fixed workspace inside the arena (split-K slices, bias-gradient
    // partials).  Captured steps bake this address in; it lives exactly as
    // long as the plan, and other plans or direct calls never touch it.
    fg_ctx wctx;
    int ws_slot = kNone;
    uint64_t ws_bytes = 0;
    std::vector<uint32_t> saved_nodes, grad_nodes;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;

    void *ptr(int slot) const {
        if (slot == kNone) return nullptr;
        const Slot &s = slots[slot];
        return s.external ? s.ext : (void *)(arena + s.offset);
    }
    // Slot of `elems` elements of type dt (bytes rounded up to whole words
    // so word fills cover it).
    int new_slot(uint64_t elems, int dt = FG_DTYPE_F32) {
        Slot s;
        s.used = elems * esize(dt);
        s.bytes = (s.used + 3) & ~uint64_t(3);
        s.dtype = dt;
        slots.push_back(s);
        return (int)slots.size() - 1;
    }
    int new_external(uint64_t elems, int dt = FG_DTYPE_F32) {
        Slot s;
        s.bytes = s.used = elems * esize(dt);
        s.dtype = dt;
        s.external = true;
        slots.push_back(s);
        return (int)slots.size() - 1;
    }
    int sdt(int slot) const { return slot == kNone ? FG_DTYPE_F32 : slots[slot].dtype; }
    int vslot(uint32_t n) const { return val_slot[n]; }
    ~fg_plan();
};

fg_plan::~fg_plan() {
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    if (mt_all) fg_mt_destroy(mt_all);
    for (fg_mt *m : mt_single)
        if (m) fg_mt_destroy(m);
    for (fg_mt *m : mt_groups)
        if (m) fg_mt_destroy(m);
    for (hipEvent_t e : events) (void)hipEventDestroy(e);
    if (side) (void)hipStreamDestroy(side);
    if (arena && ctx) {
        (void)hipSetDevice(ctx->device);
        (void)hipFree(arena);
    }
}

namespace {

// ------------------------------------------------ SaveIndicator rules
// matmul/mod.rs:191-202, softmax.rs:699-718, unary.rs:15-21,
// binary.rs:66-72 (mul/div), backend/mod.rs:1189-1208 (inputs).
void compute_saved(const fg_graph &g, const std::vector<std::vector<uint32_t>> &users,
                   std::vector<uint32_t> &save) {
    const size_t n = g.nodes.size();
    save.assign(n, 0);
    auto nonleaf = [&](uint32_t i) { return !g.nodes[i].in.empty(); };
    for (size_t i = 0; i < n; ++i) {
        const GNode &nd = g.nodes[i];
        switch (nd.op) {
            case FG_OP_INPUT: save[i] |= kDefBwd; break;
            case FG_OP_MATMUL:
                save[i] |= kDefFwd | kDefBwd;
                for (uint32_t x : nd.in)
                    if (nonleaf(x)) save[x] |= kDefFwd;
                break;
            case FG_OP_SOFTMAX:
                save[i] |= kDefFwd | kDefBwd;
                for (uint32_t x : nd.in) {
                    const int op = g.nodes[x].op;
                    if (op == FG_OP_MATMUL || op == FG_OP_GELU || op == FG_OP_SOFTMAX)
                        save[x] |= kDefFwd | kDefBwd;
                }
                for (uint32_t u : users[i]) save[u] |= kDefBwd;
                break;
            case FG_OP_MUL:
            case FG_OP_DIV:
                for (uint32_t x : nd.in)
                    if (nonleaf(x)) save[x] |= kDefFwd;
                break;
            default:
                if (is_unary(nd.op) && nonleaf(nd.in[0])) save[nd.in[0]] |= kDefFwd;
                break;
        }
    }
}

// -------------------------------------------------- elementwise batches
struct EltBuilder {
    fg_plan &P;
    Launch L;
    int nregs = 0, nsrc = 0, ndst = 0;
    int64_t numel = -1, cols = -1;
    std::vector<std::pair<uint32_t, int>> reg_of;  // node -> register in this batch
    std::vector<std::string> names;
    explicit EltBuilder(fg_plan &p) : P(p) { reset(); }
    void reset() {
        L = Launch();
        L.kind = LK_ELT;
        nregs = nsrc = ndst = 0;
        numel = cols = -1;
        reg_of.clear();
        names.clear();
    }
    bool empty() const { return L.prog.n_instr == 0; }
    int reg() { return nregs++; }
    void ins(uint8_t op, int dst, int a = 0, int b = 0, int c = 0, float imm = 0.0f) {
        fg::EltInstr &e = L.prog.ins[L.prog.n_instr++];
        e.op = op;
        e.dst = (uint8_t)dst;
        e.a = (uint8_t)a;
        e.b = (uint8_t)b;
        e.c = (uint8_t)c;
        e.imm = imm;
    }
    int find_reg(uint32_t n) const {
        for (auto &p : reg_of)
            if (p.first == n) return p.second;
        return kNone;
    }
    // Load value of node x (slot s, shape xs) into a register for an output
    // of numel/cols.
    int load(int slot, const Shape &xs) {
        const int mode = xs.scalar ? fg::kModeScalar
                         : (xs.vector && xs.numel() != numel) ? fg::kModeRow
                                                                : fg::kModeFull;
        int k = kNone;
        for (int j = 0; j < nsrc; ++j)
            if (L.src_slot[j] == slot) k = j;
        if (k == kNone) {
            k = nsrc++;
            L.src_slot[k] = slot;
        }
        const int r = reg();
        ins(fg::kEltLoad, r, k, P.sdt(slot), mode);
        return r;
    }
    // Round register r to a 16-bit node type (a node value of that type).
    void round(int r, int dt) {
        if (dt != FG_DTYPE_F32) ins(fg::kEltRound, r, r, 0, dt);
    }
    int operand(uint32_t x) {
        const GNode &nd = P.g.nodes[x];
        if (nd.op == FG_OP_CONST) {
            const int r = reg();
            ins(fg::kEltImm, r, 0, 0, 0, nd.value);
            return r;
        }
        const int r = find_reg(x);
        if (r != kNone) return r;
        return load(P.vslot(x), P.shape[x]);
    }
    void store(int slot, int r, bool accum) {
        int k = kNone;
        for (int j = 0; j < ndst; ++j)
            if (L.dst_slot[j] == slot) k = j;
        if (k == kNone) {
            k = ndst++;
            L.dst_slot[k] = slot;
        }
        ins(accum ? fg::kEltAccum : fg::kEltStore, 0, k, r, P.sdt(slot));
    }
    bool fits(int more_instr, int more_regs, int more_src, int more_dst) const {
        return L.prog.n_instr + more_instr <= fg::kEltMaxInstr &&
               nregs + more_regs <= fg::kEltRegs && nsrc + more_src <= fg::kEltMaxSrc &&
               ndst + more_dst <= fg::kEltMaxDst;
    }
    void begin(int64_t n, int64_t c) {
        numel = n;
        cols = c;
        L.prog.n = (uint64_t)n;
        L.prog.cols = (uint32_t)c;
    }
    void flush(std::vector<Launch> &out, const char *phase) {
        if (empty() || ndst == 0) {  // nothing stored: no launch
            reset();
            return;
        }
        std::string d = std::string(phase) + " eltwise[";
        for (size_t i = 0; i < names.size(); ++i) d += (i ? "," : "") + names[i];
        d += "] n=" + std::to_string(numel);
        L.desc = d;
        out.push_back(L);
        reset();
    }
};

uint8_t unary_code(int op) {
    switch (op) {
        case FG_OP_RELU: return fg::kEltRelu;
        case FG_OP_GELU: return fg::kEltGelu;
        case FG_OP_ELU: return fg::kEltElu;
        case FG_OP_TANH: return fg::kEltTanh;
        case FG_OP_EXP: return fg::kEltExp;
        case FG_OP_LOG: return fg::kEltLog;
        case FG_OP_ABS: return fg::kEltAbs;
        default: return fg::kEltNeg;
    }
}

std::string dt_suffix(int dt) {
    return dt == FG_DTYPE_F32 ? std::string() : std::string(" ") + dtype_name(dt);
}

std::string dims_str(int M, int N, int K) {
    return std::to_string(M) + "x" + std::to_string(N) + "x" + std::to_string(K);
}

// ------------------------------------------------------------ lowering
int lower_forward(fg_plan &P) {
    const fg_graph &g = P.g;
    EltBuilder eb(P);
    for (uint32_t n = 0; n < g.nodes.size(); ++n) {
        const GNode &nd = g.nodes[n];
        if (nd.op == FG_OP_INPUT || nd.op == FG_OP_CONST) continue;
        const int gi = P.group_of[n];
        if (gi != kNone) {
            const Group &G = P.groups[gi];
            if ((int)n != G.fin) continue;
            eb.flush(P.fwd, "forward");
            const uint32_t a = g.nodes[G.mm].in[0], b = g.nodes[G.mm].in[1];
            Launch L;
            L.kind = LK_GEMM;
            L.dtype = P.dtype[G.mm];
            L.layout = FG_NN;
            L.M = (int)P.shape[a].rows;
            L.K = (int)P.shape[a].cols;
            L.N = (int)P.shape[b].cols;
            L.lda = L.K;
            L.ldb = L.N;
            L.ldc = L.N;
            L.sA = P.vslot(a);
            L.sB = P.vslot(b);
            L.sBias = G.bias_src != kNone ? P.vslot(G.bias_src) : kNone;
            L.act = G.act_node == kNone ? FG_ACT_NONE
                    : g.nodes[G.act_node].op == FG_OP_RELU ? FG_ACT_RELU
                                                            : FG_ACT_GELU;
            L.sC = P.vslot(G.fin);
            L.sZ = G.act_node != kNone ? P.vslot(G.pre) : kNone;
            L.ldz = L.N;
            L.desc = "forward gemm NN " + dims_str(L.M, L.N, L.K) + dt_suffix(L.dtype) +
                     (L.sBias != kNone ? " +bias" : "") +
                     (L.act == FG_ACT_RELU ? " +relu" : L.act == FG_ACT_GELU ? " +gelu" : "") +
                     " -> node " + std::to_string(G.fin);
            P.fwd.push_back(L);
            continue;
        }
        if (nd.op == FG_OP_SOFTMAX) {
            eb.flush(P.fwd, "forward");
            Launch L;
            L.kind = LK_SOFTMAX;
            L.dtype = P.dtype[n];
            L.M = (int)P.shape[n].rows;
            L.N = (int)P.shape[n].cols;
            L.sA = P.vslot(nd.in[0]);
            L.sC = P.vslot(n);
            L.elidable = P.ce_fused_possible && (int)n == P.last;
            L.desc = "forward softmax " + std::to_string(L.M) + "x" + std::to_string(L.N) +
                     " -> node " + std::to_string(n);
            P.fwd.push_back(L);
            continue;
        }
        // elementwise node
        const Shape &s = P.shape[n];
        if (!eb.empty() && (eb.numel != s.numel() || eb.cols != s.cols || !eb.fits(7, 4, 2, 1)))
            eb.flush(P.fwd, "forward");
        if (eb.empty()) eb.begin(s.numel(), s.cols);
        int r;
        if (is_unary(nd.op)) {
            const int x = eb.operand(nd.in[0]);
            r = eb.reg();
            eb.ins(unary_code(nd.op), r, x);
        } else {
            const int x = eb.operand(nd.in[0]);
            const int y = eb.operand(nd.in[1]);
            r = eb.reg();
            const uint8_t code = (nd.op == FG_OP_ADD || nd.op == FG_OP_BIAS_ADD) ? fg::kEltAdd
                                 : nd.op == FG_OP_SUB                          ? fg::kEltSub
                                 : nd.op == FG_OP_MUL                          ? fg::kEltMul
                                                                               : fg::kEltDiv;
            eb.ins(code, r, x, y);
        }
        eb.round(r, P.dtype[n]);
        eb.reg_of.push_back({n, r});
        eb.store(P.vslot(n), r, false);
        eb.names.push_back(std::string(op_name(nd.op)) + "#" + std::to_string(n));
    }
    eb.flush(P.fwd, "forward");
    // Forward GEMM chains (the first's output is the next's A operand).
    for (size_t i = 0; i + 1 < P.fwd.size(); ++i) {
        Launch &L = P.fwd[i];
        const Launch &X = P.fwd[i + 1];
        const bool gemm = L.kind == LK_GEMM && X.kind == LK_GEMM && L.sExtra == kNone &&
                          X.sExtra == kNone && L.dtype == FG_DTYPE_F32 &&
                          X.dtype == FG_DTYPE_F32 && L.layout == FG_NN && X.layout == FG_NN;
        if (gemm && X.sA == L.sC && X.lda == L.ldc && X.K == L.N && X.M == L.M &&
            !L.accumulate) {
            L.chain_next = true;  // described where it chains (fg_plan_describe)
            ++i;                  // a launch is the second of at most one chain
        }
    }
    return FG_OK;
}

int lower_loss(fg_plan &P) {
    const fg_graph &g = P.g;
    const uint32_t last = (uint32_t)P.last;
    const Shape &s = P.shape[last];
    if (P.ce_fused_possible) {
        const uint32_t x = g.nodes[last].in[0];
        Launch L;
        L.kind = LK_SMCE;
        L.dtype = P.dtype[x];
        L.M = (int)s.rows;
        L.N = (int)s.cols;
        L.sA = P.vslot(x);
        L.sZ = P.target_slot;  // labels
        L.sB = P.loss_slot;    // row loss
        L.sBias = P.mean_slot;
        L.sC = P.needs_grad[x] ? P.grad_slot[x] : kNone;
        L.sProbs = P.vslot(last);
        L.desc = "loss softmax+ce " + std::to_string(L.M) + "x" + std::to_string(L.N) +
                 " (dlogits -> grad of node " + std::to_string(x) + ")";
        P.loss.push_back(L);
        return FG_OK;
    }
    EltBuilder eb(P);
    eb.begin(s.numel(), s.cols);
    const int p = eb.load(P.vslot(last), s);
    const int seed = P.grad_slot[last];
    if (g.loss == FG_LOSS_CE) {
        // basic_loss.rs:91-133: grad = p - [col == label]; loss = -log p at
        // the label column, 0 elsewhere.
        eb.L.label_slot = P.target_slot;
        const int oh = eb.reg();
        eb.ins(fg::kEltLabelEq, oh);
        const int gr = eb.reg();
        eb.ins(fg::kEltSub, gr, p, oh);
        eb.store(seed, gr, false);
        const int lp = eb.reg();
        eb.ins(fg::kEltLog, lp, p);
        const int nl = eb.reg();
        eb.ins(fg::kEltNeg, nl, lp);
        const int z = eb.reg();
        eb.ins(fg::kEltImm, z, 0, 0, 0, 0.0f);
        const int lo = eb.reg();
        eb.ins(fg::kEltSelect, lo, oh, nl, z);
        eb.store(P.loss_slot, lo, false);
        eb.names.push_back("ce");
    } else {
        Shape ts = s;
        const int t = eb.load(P.target_slot, ts);
        const int d = eb.reg();
        eb.ins(fg::kEltSub, d, p, t);
        if (g.loss == FG_LOSS_MSE) {
            // basic_loss.rs:3-27: loss = (p-t)^2, grad = 2(p-t)
            const int l = eb.reg();
            eb.ins(fg::kEltMul, l, d, d);
            eb.store(P.loss_slot, l, false);
            const int two = eb.reg();
            eb.ins(fg::kEltImm, two, 0, 0, 0, 2.0f);
            const int gr = eb.reg();
            eb.ins(fg::kEltMul, gr, two, d);
            eb.store(seed, gr, false);
            eb.names.push_back("mse");
        } else {
            // basic_loss.rs:29-89: loss = -(t log p + (1-t) log(1-p)) (the
            // reference takes 1-t for 1-p -- corrected), grad = p - t.
            const int one = eb.reg();
            eb.ins(fg::kEltImm, one, 0, 0, 0, 1.0f);
            const int lp = eb.reg();
            eb.ins(fg::kEltLog, lp, p);
            const int omp = eb.reg();
            eb.ins(fg::kEltSub, omp, one, p);
            const int lomp = eb.reg();
            eb.ins(fg::kEltLog, lomp, omp);
            const int omt = eb.reg();
            eb.ins(fg::kEltSub, omt, one, t);
            const int t1 = eb.reg();
            eb.ins(fg::kEltMul, t1, t, lp);
            const int t2 = eb.reg();
            eb.ins(fg::kEltMul, t2, omt, lomp);
            eb.ins(fg::kEltAdd, t1, t1, t2);
            eb.ins(fg::kEltNeg, t1, t1);
            eb.store(P.loss_slot, t1, false);
            eb.store(seed, d, false);
            eb.names.push_back("bce");
        }
    }
    eb.flush(P.loss, "loss");
    return FG_OK;
}

// Backward for one mode.  fused: the loss kernel already wrote the CE
// gradient of the final softmax's input; otherwise start from the seed.
int lower_backward(fg_plan &P, bool fused, std::vector<Launch> &out) {
    const fg_graph &g = P.g;
    const size_t nn = g.nodes.size();
    std::vector<char> ginit(nn, 0), gskip(nn, 0);
    const uint32_t last = (uint32_t)P.last;
    if (fused)
        ginit[g.nodes[last].in[0]] = 1;
    else
        ginit[last] = 1;
    auto gs = [&](uint32_t n) { return P.grad_slot[n]; };
    EltBuilder eb(P);
    auto elt_contrib = [&](uint32_t n) {
        // One program per elementwise node: contributions to its inputs.
        const GNode &nd = g.nodes[n];
        const Shape &s = P.shape[n];
        eb.begin(s.numel(), s.cols);
        const int gr = eb.load(gs(n), s);
        auto emit = [&](uint32_t x, int r) {
            if (!P.needs_grad[x]) return;
            eb.store(gs(x), r, ginit[x] != 0);
            ginit[x] = 1;
        };
        const int op = nd.op;
        if (is_unary(op)) {
            const uint32_t x = nd.in[0];
            if (!P.needs_grad[x]) {
                eb.reset();
                return;
            }
            int d;
            switch (op) {
                case FG_OP_NEG: d = eb.reg(); eb.ins(fg::kEltNeg, d, gr); break;
                case FG_OP_TANH: {  // 1 - y^2 (y = output)
                    const int y = eb.load(P.vslot(n), s);
                    const int y2 = eb.reg(); eb.ins(fg::kEltMul, y2, y, y);
                    const int one = eb.reg(); eb.ins(fg::kEltImm, one, 0, 0, 0, 1.0f);
                    const int dd = eb.reg(); eb.ins(fg::kEltSub, dd, one, y2);
                    d = eb.reg(); eb.ins(fg::kEltMul, d, gr, dd);
                    break;
                }
                case FG_OP_EXP: {  // y
                    const int y = eb.load(P.vslot(n), s);
                    d = eb.reg(); eb.ins(fg::kEltMul, d, gr, y);
                    break;
                }
                case FG_OP_LOG: {  // 1/x (the reference divides by its output, unary.rs:241-249)
                    const int xv = eb.operand(x);
                    d = eb.reg(); eb.ins(fg::kEltDiv, d, gr, xv);
                    break;
                }
                default: {  // relu, gelu, elu, abs: g * f'(x)
                    const int xv = eb.operand(x);
                    const uint8_t code = op == FG_OP_RELU ? fg::kEltReluD
                                         : op == FG_OP_GELU ? fg::kEltGeluD
                                         : op == FG_OP_ELU ? fg::kEltEluD
                                                           : fg::kEltSign;
                    const int dd = eb.reg(); eb.ins(code, dd, xv);
                    d = eb.reg(); eb.ins(fg::kEltMul, d, gr, dd);
                    break;
                }
            }
            emit(x, d);
        } else {
            const uint32_t a = nd.in[0], b = nd.in[1];
            const Shape &sa = P.shape[a], &sb = P.shape[b];
            const bool bcast_a = !sa.scalar && sa.numel() != s.numel();
            const bool bcast_b = !sb.scalar && sb.numel() != s.numel();
            // Row-broadcast operands reduce over rows: handled by bias_grad
            // for add/sub; products with a broadcast vector are rejected at
            // plan creation.
            if (op == FG_OP_ADD || op == FG_OP_BIAS_ADD || op == FG_OP_SUB) {
                if (P.needs_grad[a] && !bcast_a) emit(a, gr);
                if (P.needs_grad[b] && !bcast_b) {
                    if (op == FG_OP_SUB) {
                        const int d = eb.reg(); eb.ins(fg::kEltNeg, d, gr);
                        emit(b, d);
                    } else {
                        emit(b, gr);
                    }
                }
            } else if (op == FG_OP_MUL) {
                if (P.needs_grad[a]) {
                    const int bv = eb.operand(b);
                    const int d = eb.reg(); eb.ins(fg::kEltMul, d, gr, bv);
                    emit(a, d);
                }
                if (P.needs_grad[b]) {
                    const int av = eb.operand(a);
                    const int d = eb.reg(); eb.ins(fg::kEltMul, d, gr, av);
                    emit(b, d);
                }
            } else {  // DIV: d/da = g / b ; d/db = -g a / b^2
                const int bv = eb.operand(b);
                if (P.needs_grad[a]) {
                    const int d = eb.reg(); eb.ins(fg::kEltDiv, d, gr, bv);
                    emit(a, d);
                }
                if (P.needs_grad[b]) {
                    const int av = eb.operand(a);
                    const int q = eb.reg(); eb.ins(fg::kEltDiv, q, av, bv);
                    const int q2 = eb.reg(); eb.ins(fg::kEltDiv, q2, q, bv);
                    const int d0 = eb.reg(); eb.ins(fg::kEltMul, d0, gr, q2);
                    const int d = eb.reg(); eb.ins(fg::kEltNeg, d, d0);
                    emit(b, d);
                }
            }
            eb.names.push_back(std::string("d") + op_name(op) + "#" + std::to_string(n));
            eb.flush(out, "backward");
            // Column reductions for broadcast operands.
            auto reduce = [&](uint32_t x, bool neg) {
                if (!P.needs_grad[x]) return;
                Launch L;
                L.kind = LK_BIAS_GRAD;
                L.dtype = P.sdt(gs(n));
                L.M = (int)s.rows;
                L.N = (int)s.cols;
                L.sA = gs(n);
                L.desc = "backward bias_grad " + std::to_string(L.M) + "x" + std::to_string(L.N);
                if (!neg) {
                    L.sC = gs(x);
                    L.accumulate = ginit[x];
                    L.desc += " -> grad of node " + std::to_string(x);
                    ginit[x] = 1;
                    out.push_back(L);
                    return;
                }
                // sub's broadcast operand: reduce into a temporary, then
                // grad (=|+=) -temporary.
                const int tmp = P.new_slot((uint64_t)L.N, L.dtype);
                L.sC = tmp;
                L.desc += " -> temporary";
                out.push_back(L);
                Shape vs;
                vs.vector = true;
                vs.cols = L.N;
                eb.begin(L.N, L.N);
                const int t = eb.load(tmp, vs);
                const int d = eb.reg();
                eb.ins(fg::kEltNeg, d, t);
                eb.store(gs(x), d, ginit[x] != 0);
                ginit[x] = 1;
                eb.names.push_back("neg-reduce#" + std::to_string(x));
                eb.flush(out, "backward");
            };
            if (bcast_a) reduce(a, false);
            if (bcast_b) reduce(b, op == FG_OP_SUB);
            return;
        }
        eb.names.push_back(std::string("d") + op_name(op) + "#" + std::to_string(n));
        eb.flush(out, "backward");
    };

    for (int64_t ni = (int64_t)nn - 1; ni >= 0; --ni) {
        const uint32_t n = (uint32_t)ni;
        const GNode &nd = g.nodes[n];
        if (nd.op == FG_OP_INPUT || nd.op == FG_OP_CONST || !P.needs_grad[n]) continue;
        if (fused && n == last) continue;
        const int gi = P.group_of[n];
        if (gi != kNone) {
            const Group &G = P.groups[gi];
            if ((int)n != G.fin) continue;
            const int pre = G.pre;
            if (G.act_node != kNone && !gskip[G.act_node]) {
                if (!ginit[G.act_node]) continue;
                // dZ = dH * act'(Z) as a program (no downstream GEMM took it).
                const Shape &s = P.shape[pre];
                eb.begin(s.numel(), s.cols);
                const int gh = eb.load(gs(G.act_node), s);
                const int z = eb.load(P.vslot(pre), s);
                const int dd = eb.reg();
                eb.ins(g.nodes[G.act_node].op == FG_OP_RELU ? fg::kEltReluD : fg::kEltGeluD, dd, z);
                const int d = eb.reg();
                eb.ins(fg::kEltMul, d, gh, dd);
                eb.store(gs(pre), d, ginit[pre] != 0);
                ginit[pre] = 1;
                eb.names.push_back("dact#" + std::to_string(G.act_node));
                eb.flush(out, "backward");
            } else if (G.act_node == kNone && !ginit[pre]) {
                continue;
            }
            const uint32_t a = g.nodes[G.mm].in[0], b = g.nodes[G.mm].in[1];
            const int M = (int)P.shape[a].rows, K = (int)P.shape[a].cols, N = (int)P.shape[b].cols;
            // The bias gradient rides on the dW GEMM (column sums of dZ from
            // its B tiles) when that GEMM runs and dZ and the bias share its
            // element type.
            const bool fuse_db = G.bias_src != kNone && P.needs_grad[G.bias_src] &&
                                 P.needs_grad[b] && P.sdt(gs(G.bias_src)) == P.dtype[G.mm] &&
                                 P.sdt(gs(pre)) == P.dtype[G.mm];
            if (G.bias_src != kNone && P.needs_grad[G.bias_src] && !fuse_db) {
                Launch L;
                L.kind = LK_BIAS_GRAD;
                L.dtype = P.sdt(gs(pre));
                L.M = M;
                L.N = N;
                L.sA = gs(pre);
                L.sC = gs(G.bias_src);
                L.accumulate = ginit[G.bias_src];
                L.desc = "backward bias_grad " + std::to_string(M) + "x" + std::to_string(N) +
                         " -> grad of node " + std::to_string(G.bias_src);
                ginit[G.bias_src] = 1;
                out.push_back(L);
            }
            int idx_db = kNone;
            if (P.needs_grad[b]) {  // dB = A^T dZ
                idx_db = (int)out.size();
                Launch L;
                L.kind = LK_GEMM;
                L.dtype = P.dtype[G.mm];
                L.layout = FG_TN;
                L.M = K;
                L.N = N;
                L.K = M;
                L.sA = P.vslot(a);
                L.lda = K;
                L.sB = gs(pre);
                L.ldb = N;
                L.sC = gs(b);
                L.ldc = N;
                L.accumulate = ginit[b];
                L.desc = "backward gemm TN " + dims_str(K, N, M) + " -> grad of node " +
                         std::to_string(b);
                ginit[b] = 1;
                if (fuse_db) {
                    L.sExtra = gs(G.bias_src);
                    L.accumulate2 = ginit[G.bias_src];
                    ginit[G.bias_src] = 1;
                    L.desc += " +dbias -> grad of node " + std::to_string(G.bias_src);
                }
                out.push_back(L);
            }
            if (P.needs_grad[a]) {  // dA = dZ B^T  (with act' of the layer below fused)
                Launch L;
                L.kind = LK_GEMM_BWD;
                L.dtype = P.dtype[G.mm];
                L.layout = FG_NT;
                L.M = M;
                L.N = K;
                L.K = N;
                L.sA = gs(pre);
                L.lda = N;
                L.sB = P.vslot(b);
                L.ldb = N;
                L.ldc = K;
                const int ga = P.group_of[a];
                const bool fuse = ga != kNone && P.groups[ga].act_node == (int)a &&
                                  P.users[a].size() == 1 && !ginit[a];
                if (fuse) {
                    const Group &G2 = P.groups[ga];
                    L.act = g.nodes[a].op == FG_OP_RELU ? FG_ACT_RELU : FG_ACT_GELU;
                    L.sZ = P.vslot(G2.pre);
                    L.ldz = K;
                    L.sC = gs(G2.pre);
                    L.accumulate = ginit[G2.pre];
                    ginit[G2.pre] = 1;
                    gskip[a] = 1;
                    L.desc = "backward gemm NT " + dims_str(M, K, N) + " *" +
                             (L.act == FG_ACT_RELU ? "relu'" : "gelu'") + " -> grad of node " +
                             std::to_string(G2.pre);
                } else {
                    L.sC = gs(a);
                    L.accumulate = ginit[a];
                    ginit[a] = 1;
                    L.desc = "backward gemm NT " + dims_str(M, K, N) + " -> grad of node " +
                             std::to_string(a);
                }
                if (idx_db != kNone && a != b) {
                    out[idx_db].pair_next = true;
                    out[idx_db].desc += " [with the next]";
                }
                out.push_back(L);
            }
            continue;
        }
        if (!ginit[n]) continue;  // no gradient reaches this node
        if (nd.op == FG_OP_SOFTMAX) {
            const uint32_t x = nd.in[0];
            if (!P.needs_grad[x]) continue;
            Launch L;
            L.kind = LK_SOFTMAX_BWD;
            L.dtype = P.dtype[n];
            L.M = (int)P.shape[n].rows;
            L.N = (int)P.shape[n].cols;
            L.sA = P.vslot(n);
            L.sB = gs(n);
            L.sC = gs(x);
            L.accumulate = ginit[x];
            ginit[x] = 1;
            L.desc = "backward softmax " + std::to_string(L.M) + "x" + std::to_string(L.N) +
                     " -> grad of node " + std::to_string(x);
            out.push_back(L);
            continue;
        }
        elt_contrib(n);
    }
    // Inputs no gradient reached get zeros.
    for (uint32_t n : P.inputs) {
        if (!P.needs_grad[n] || ginit[n]) continue;
        Launch L;
        L.kind = LK_FILL0;
        L.sC = gs(n);
        L.count = P.slots[gs(n)].bytes / 4;  // words (slot sizes are whole words)
        L.desc = "backward zero grad of node " + std::to_string(n);
        out.push_back(L);
    }
    return FG_OK;
}

// ------------------------------------------------------- static checks
int check_slot(const fg_plan &P, const Launch &L, int slot, uint64_t need, const char *what) {
    if (slot == kNone) return FG_OK;
    FG_REQUIRE(slot >= 0 && slot < (int)P.slots.size(), FG_ERR_INTERNAL,
               "plan: %s of '%s' refers to slot %d of %zu", what, L.desc.c_str(), slot,
               P.slots.size());
    FG_REQUIRE(P.slots[slot].bytes >= need, FG_ERR_INTERNAL,
               "plan: %s of '%s' needs %llu bytes, slot %d has %llu", what, L.desc.c_str(),
               (unsigned long long)need, slot, (unsigned long long)P.slots[slot].bytes);
    return FG_OK;
}

int check_launch(const fg_plan &P, const Launch &L) {
    const uint64_t M = (uint64_t)L.M, N = (uint64_t)L.N, K = (uint64_t)L.K;
    int rc = FG_OK;
    // elems of the slot's own element type (fill counts are words).
    auto chk = [&](int slot, uint64_t elems, const char *what) {
        if (rc == FG_OK && slot != kNone)
            rc = check_slot(P, L, slot,
                            elems * (L.kind == LK_FILL0 ? 4 : esize(P.slots[slot].dtype)), what);
    };
    switch (L.kind) {
        case LK_GEMM:
        case LK_GEMM_BWD:
            chk(L.sA, M * K, "A");
            chk(L.sB, K * N, "B");
            chk(L.sC, M * N, "C");
            chk(L.sZ, M * N, "Z");
            chk(L.sBias, N, "bias");
            chk(L.sExtra, N, "dbias");
            break;
        case LK_BIAS_GRAD:
            chk(L.sA, M * N, "dZ");
            chk(L.sC, N, "dbias");
            break;
        case LK_SOFTMAX:
        case LK_SOFTMAX_BWD:
            chk(L.sA, M * N, "x");
            chk(L.sB, M * N, "dy");
            chk(L.sC, M * N, "out");
            break;
        case LK_SMCE:
            chk(L.sA, M * N, "logits");
            chk(L.sZ, M, "labels");
            chk(L.sB, M, "row loss");
            chk(L.sBias, 1, "mean loss");
            chk(L.sC, M * N, "dlogits");
            chk(L.sProbs, M * N, "probabilities");
            break;
        case LK_FILL0:
            chk(L.sC, L.count, "fill");
            break;
        case LK_ELT: {
            const fg::EltProgram &p = L.prog;
            FG_REQUIRE(p.n_instr > 0 && p.n_instr <= fg::kEltMaxInstr, FG_ERR_INTERNAL,
                       "plan: '%s' has %d instructions", L.desc.c_str(), p.n_instr);
            for (int k = 0; k < p.n_instr && rc == FG_OK; ++k) {
                const fg::EltInstr &in = p.ins[k];
                FG_REQUIRE(in.dst < fg::kEltRegs && in.a < 16 && in.b < 16 && in.c < 16,
                           FG_ERR_INTERNAL, "plan: '%s' instruction %d out of range",
                           L.desc.c_str(), k);
                if (in.op == fg::kEltLoad) {
                    FG_REQUIRE(in.a < fg::kEltMaxSrc && L.src_slot[in.a] != kNone,
                               FG_ERR_INTERNAL, "plan: '%s' loads unset source %d",
                               L.desc.c_str(), in.a);
                    const uint8_t mode = in.c;
                    FG_REQUIRE(mode <= fg::kModeScalar, FG_ERR_INTERNAL,
                               "plan: '%s' load with mode %d", L.desc.c_str(), mode);
                    chk(L.src_slot[in.a],
                        mode == fg::kModeScalar ? 1 : mode == fg::kModeRow ? p.cols : p.n,
                        "source");
                } else if (in.op == fg::kEltStore || in.op == fg::kEltAccum) {
                    FG_REQUIRE(in.a < fg::kEltMaxDst && L.dst_slot[in.a] != kNone,
                               FG_ERR_INTERNAL, "plan: '%s' stores to unset destination %d",
                               L.desc.c_str(), in.a);
                    chk(L.dst_slot[in.a], p.n, "destination");
                } else if (in.op == fg::kEltLabelEq) {
                    FG_REQUIRE(p.cols > 0 && L.label_slot != kNone, FG_ERR_INTERNAL,
                               "plan: '%s' compares labels without labels", L.desc.c_str());
                    chk(L.label_slot, p.n / p.cols, "labels");
                }
            }
            break;
        }
        default:
            break;
    }
    return rc;
}

// ------------------------------------------------------------ execute
// step: the launches belong to a whole captured step (forward through
// optimiser), so the final forward softmax is left to the loss launch.
// The loss of a captured SGD step finished in its head GEMM: the plan's one
// loss launch, an fp32 softmax + CE on the 16-lane row path, whose logits
// are the whole output of the second GEMM of a forward chain.  Returns the
// index in fwd of the chain's first launch, or -1.  (Whether the chain
// chains is decided when it runs, fg::gemm_fwd_chain_f32.)
int head_loss_chain(const fg_plan &P) {
    if (P.g.optim != FG_OPTIM_SGD || P.opt_inputs.empty() || P.loss.size() != 1) return -1;
    const Launch &S = P.loss[0];
    if (S.kind != LK_SMCE || S.dtype != FG_DTYPE_F32 || !fg::softmax_ce_row16_case(S.M, S.N))
        return -1;
    for (size_t i = 0; i + 1 < P.fwd.size(); ++i) {
        const Launch &L = P.fwd[i], &X = P.fwd[i + 1];
        if (L.chain_next && X.sC == S.sA && X.act == FG_ACT_NONE && !X.accumulate &&
            X.M == S.M && X.N == S.N && X.ldc == S.N)
            return (int)i;
    }
    return -1;
}

// With the loss finished in the head GEMM (head_loss_chain, chain at fwd
// index hc), the head kernel can also compute the backward's data gradient
// of the head, dZ = (dlogits . W^T) * act'(Z): when the backward list opens
// with the head's dW (+ dbias, paired with that dX, fp32) and the dX reads
// the loss's dlogits and the head's weight, writes a whole fresh gradient
// (no accumulation) through act' of the summed GEMM's Z, and takes a 64x64
// tile kernel (more than 16 output columns).  The backward then runs the
// head's dW with the next pair in one launch (run's triple_at = 0).
bool head_bwd_fusable(const fg_plan &P, const std::vector<Launch> &bwd, int hc) {
    if (hc < 0 || bwd.size() < 4) return false;
    const Launch &S = P.loss[0], &L = P.fwd[hc], &X = P.fwd[hc + 1];
    const Launch &W0 = bwd[0], &D0 = bwd[1], &W1 = bwd[2], &D1 = bwd[3];
    const bool dw0 = W0.kind == LK_GEMM && W0.sExtra != kNone && W0.dtype == FG_DTYPE_F32 &&
                     W0.pair_next && W0.sA == X.sA && W0.sB == S.sC;
    const bool dx0 = D0.kind == LK_GEMM_BWD && D0.layout == FG_NT && D0.dtype == FG_DTYPE_F32 &&
                     D0.sA == S.sC && D0.sB == X.sB && D0.M == S.M && D0.N == X.K &&
                     D0.K == S.N && D0.N > fg::gemm_skinny_max_n() && !D0.accumulate &&
                     D0.ldc == D0.N && D0.lda == S.N && D0.ldb == X.ldb &&
                     (D0.act == FG_ACT_NONE || (D0.sZ == L.sZ && D0.ldz == D0.N && L.ldz == L.N));
    const bool pair1 = W1.kind == LK_GEMM && W1.sExtra != kNone && W1.dtype == FG_DTYPE_F32 &&
                       W1.pair_next && D1.kind == LK_GEMM_BWD && D1.dtype == FG_DTYPE_F32;
    return dw0 && dx0 && pair1;
}

// The elementwise program of an LK_ELT launch with the plan's pointers.
int elt_program(const fg_plan &P, const Launch &L, fg::EltProgram *out) {
    fg::EltProgram &p = *out;
    p = L.prog;
    for (int k = 0; k < fg::kEltMaxSrc; ++k)
        if (L.src_slot[k] != kNone) {
            p.src[k] = (const float *)P.ptr(L.src_slot[k]);
            FG_REQUIRE(p.src[k], FG_ERR_INVALID_ARGUMENT, "plan: unbound input or target (%s)",
                       L.desc.c_str());
        }
    for (int k = 0; k < fg::kEltMaxDst; ++k)
        if (L.dst_slot[k] != kNone) p.dst[k] = (float *)P.ptr(L.dst_slot[k]);
    if (L.label_slot != kNone) {
        p.labels = (const uint32_t *)P.ptr(L.label_slot);
        FG_REQUIRE(p.labels, FG_ERR_INVALID_ARGUMENT,
                   "dispatch_loss: no target bound (fg_plan_bind_target)");
    }
    return FG_OK;
}

// Compiles, ahead of a stream capture, the elementwise kernels that the
// lists' programs will take (a capture meeting one not compiled yet would
// run it on the interpreter).
int prepare_elt(fg_plan &P, std::initializer_list<const std::vector<Launch> *> lists) {
    for (const std::vector<Launch> *list : lists)
        for (const Launch &L : *list) {
            if (L.kind != LK_ELT) continue;
            fg::EltProgram p;
            if (int rc = elt_program(P, L, &p)) return rc;
            if (int rc = fg::prepare_eltwise(&P.wctx, p)) return rc;
        }
    return FG_OK;
}

// defer_last: the summing launch of a split GEMM in the list's last launch
// (or the pair or chain ending it) is held in the plan's context view for the
// optimiser launch that follows (captured steps, run_optim).  ce_loss: the
// loss launch that the chain producing its logits may finish (head_loss_chain);
// *ce_done tells whether it did.
// dz_launch: with ce_loss, the backward's data-gradient launch of the head
// that the chained head kernel computes as well (head_bwd_fusable).
// triple_at: index of a head's weight-gradient launch whose group runs as
// one launch with the pair two launches on (its own pair partner, the
// head's data gradient, was computed in the forward).
// after_group (optional) runs after each launch group with the index of
// its last launch (captured Adam steps hang the optimiser's grouped updates
// there).
int run(fg_plan &P, const std::vector<Launch> &list, bool step = false, bool defer_last = false,
        const Launch *ce_loss = nullptr, bool *ce_done = nullptr,
        const Launch *dz_launch = nullptr, int triple_at = -1,
        const std::function<int(size_t)> *after_group = nullptr) {
    fg_ctx *ctx = &P.wctx;
    int skip = 0;  // launches already run as part of a group
    size_t group_end = 0;  // last launch of the group started most recently
    bool pending = false;
    for (size_t i = 0; i < list.size(); ++i) {
        const Launch &L = list[i];
        int rc = FG_OK;
        if (pending && i > group_end) {
            pending = false;
            if (int r = (*after_group)(group_end)) return r;
        }
        if (skip > 0) {
            --skip;
            continue;
        }
        size_t last = i;  // the group's last launch
        if ((int)i == triple_at && i + 3 < list.size())
            last = i + 3;
        else if ((L.pair_next || L.chain_next) && i + 1 < list.size())
            last = i + 1;
        ctx->defer_reduce = defer_last && last == list.size() - 1;
        group_end = last;
        pending = after_group != nullptr;
        if (step && L.elidable) continue;
        if ((int)i == triple_at && i + 3 < list.size()) {
            const Launch &W = list[i + 2], &X = list[i + 3];  // a layer's dW (TN) and dX (NT)
            rc = fg::gemm_dw_dw_dx_f32(
                ctx, L.M, L.N, L.K, (const float *)P.ptr(L.sA), L.lda, (const float *)P.ptr(L.sB),
                L.ldb, (float *)P.ptr(L.sC), L.ldc, L.accumulate, (float *)P.ptr(L.sExtra),
                L.accumulate2, W.M, W.N, W.K, (const float *)P.ptr(W.sA), W.lda,
                (const float *)P.ptr(W.sB), W.ldb, (float *)P.ptr(W.sC), W.ldc, W.accumulate,
                (float *)P.ptr(W.sExtra), W.accumulate2, X.M, X.N, X.K, (const float *)P.ptr(X.sA),
                X.lda, (const float *)P.ptr(X.sB), X.ldb, X.act, (const float *)P.ptr(X.sZ), X.ldz,
                (float *)P.ptr(X.sC), X.ldc, X.accumulate);
            if (rc != FG_OK) return rc;
            skip = 3;
            continue;
        }
        if (L.chain_next && i + 1 < list.size()) {
            const Launch &X = list[i + 1];  // reads L's output as its A operand
            fg::CeOut ce{};
            const bool want_ce = ce_loss && ce_done && X.sC == ce_loss->sA;
            if (want_ce) {
                const Launch &S = *ce_loss;
                FG_REQUIRE(P.ptr(S.sZ), FG_ERR_INVALID_ARGUMENT,
                           "dispatch_loss: no target bound (fg_plan_bind_target)");
                ce = {(const uint32_t *)P.ptr(S.sZ), (float *)P.ptr(S.sB), (float *)P.ptr(S.sC),
                      step ? (float *)P.ptr(S.sProbs) : nullptr, S.N, S.N, 1.0f,
                      dz_launch ? (float *)P.ptr(dz_launch->sC) : nullptr,
                      dz_launch ? dz_launch->ldc : 0, dz_launch ? dz_launch->act : FG_ACT_NONE};
            }
            rc = fg::gemm_fwd_chain_f32(
                ctx, L.M, L.N, L.K, (const float *)P.ptr(L.sA), L.lda, (const float *)P.ptr(L.sB),
                L.ldb, (const float *)P.ptr(L.sBias), L.act, (float *)P.ptr(L.sC), L.ldc,
                (float *)P.ptr(L.sZ), L.ldz, X.M, X.N, X.K, (const float *)P.ptr(X.sA), X.lda,
                (const float *)P.ptr(X.sB), X.ldb, (const float *)P.ptr(X.sBias), X.act,
                (float *)P.ptr(X.sC), X.ldc, (float *)P.ptr(X.sZ), X.ldz, X.accumulate,
                want_ce ? &ce : nullptr, want_ce ? ce_done : nullptr);
            if (rc != FG_OK) return rc;
            skip = 1;
            continue;
        }
        if (L.pair_next && i + 1 < list.size() && L.dtype != FG_DTYPE_F32) {
            const Launch &X = list[i + 1];  // the same layer's dX (NT, act'), 16-bit
            rc = fg::gemm16_dw_dx(ctx, L.dtype, L.M, L.N, L.K, P.ptr(L.sA), L.lda, P.ptr(L.sB),
                                  L.ldb, P.ptr(L.sC), L.ldc, L.accumulate, P.ptr(L.sExtra),
                                  L.accumulate2, X.M, X.N, X.K, P.ptr(X.sA), X.lda, P.ptr(X.sB),
                                  X.ldb, X.act, P.ptr(X.sZ), X.ldz, P.ptr(X.sC), X.ldc,
                                  X.accumulate);
            if (rc != FG_OK) return rc;
            skip = 1;
            continue;
        }
        if (L.pair_next && i + 1 < list.size()) {
            const Launch &X = list[i + 1];  // the same layer's dX (NT, act')
            rc = fg::gemm_dw_dx_f32(ctx, L.M, L.N, L.K, (const float *)P.ptr(L.sA), L.lda,
                                    (const float *)P.ptr(L.sB), L.ldb, (float *)P.ptr(L.sC),
                                    L.ldc, L.accumulate, (float *)P.ptr(L.sExtra), L.accumulate2,
                                    X.M, X.N, X.K, (const float *)P.ptr(X.sA), X.lda,
                                    (const float *)P.ptr(X.sB), X.ldb, X.act,
                                    (const float *)P.ptr(X.sZ), X.ldz, (float *)P.ptr(X.sC),
                                    X.ldc, X.accumulate);
            if (rc != FG_OK) return rc;
            skip = 1;
            continue;
        }
        switch (L.kind) {
            case LK_GEMM:
                if (L.sExtra != kNone && L.dtype == FG_DTYPE_F32)  // dW with the fused dbias (TN)
                    rc = fg_gemm_dw_f32(ctx, L.M, L.N, L.K, (const float *)P.ptr(L.sA), L.lda,
                                        (const float *)P.ptr(L.sB), L.ldb, (float *)P.ptr(L.sC),
                                        L.ldc, L.accumulate, (float *)P.ptr(L.sExtra),
                                        L.accumulate2);
                else if (L.sExtra != kNone)
                    rc = fg_gemm_dw_x16(ctx, L.dtype, L.M, L.N, L.K, P.ptr(L.sA), L.lda,
                                        P.ptr(L.sB), L.ldb, P.ptr(L.sC), L.ldc, L.accumulate,
                                        P.ptr(L.sExtra), L.accumulate2);
                else if (L.dtype == FG_DTYPE_F32)
                    rc = fg_gemm_f32(ctx, L.layout, L.M, L.N, L.K, (const float *)P.ptr(L.sA),
                                     L.lda, (const float *)P.ptr(L.sB), L.ldb,
                                     (const float *)P.ptr(L.sBias), L.act, (float *)P.ptr(L.sC),
                                     L.ldc, (float *)P.ptr(L.sZ), L.ldz, L.accumulate);
                else
                    rc = fg_gemm_x16(ctx, L.dtype, L.layout, L.M, L.N, L.K, P.ptr(L.sA), L.lda,
                                     P.ptr(L.sB), L.ldb, P.ptr(L.sBias), L.act, P.ptr(L.sC),
                                     L.ldc, P.ptr(L.sZ), L.ldz, L.accumulate);
                break;
            case LK_GEMM_BWD:
                if (L.dtype == FG_DTYPE_F32)
                    rc = fg_gemm_bwd_f32(ctx, L.layout, L.M, L.N, L.K,
                                         (const float *)P.ptr(L.sA), L.lda,
                                         (const float *)P.ptr(L.sB), L.ldb, L.act,
                                         (const float *)P.ptr(L.sZ), L.ldz,
                                         (float *)P.ptr(L.sC), L.ldc, L.accumulate);
                else
                    rc = fg_gemm_bwd_x16(ctx, L.dtype, L.layout, L.M, L.N, L.K, P.ptr(L.sA),
                                         L.lda, P.ptr(L.sB), L.ldb, L.act, P.ptr(L.sZ), L.ldz,
                                         P.ptr(L.sC), L.ldc, L.accumulate);
                break;
            case LK_BIAS_GRAD:
                rc = fg_bias_grad(ctx, L.dtype, L.M, L.N, P.ptr(L.sA), L.N, P.ptr(L.sC),
                                  L.accumulate);
                break;
            case LK_SOFTMAX:
                rc = fg_softmax(ctx, L.dtype, P.ptr(L.sA), L.M, L.N, P.ptr(L.sC));
                break;
            case LK_SOFTMAX_BWD:
                rc = fg_softmax_bwd(ctx, L.dtype, P.ptr(L.sA), P.ptr(L.sB), L.M, L.N, P.ptr(L.sC),
                                    L.accumulate);
                break;
            case LK_SMCE: {
                FG_REQUIRE(P.ptr(L.sZ), FG_ERR_INVALID_ARGUMENT,
                           "dispatch_loss: no target bound (fg_plan_bind_target)");
                // A captured Adam step leaves the mean loss, a launch of its
                // own here, to its second stream (run_bwd_adam_overlapped).
                const bool hold = P.hold_mean && fg::softmax_ce_dispatches(L.M, L.N, true) == 2;
                float *mean = (float *)P.ptr(L.sBias);
                rc = fg::softmax_ce_ex(ctx, L.dtype, P.ptr(L.sA), L.N,
                                       (const uint32_t *)P.ptr(L.sZ), L.M, L.N, 1.0f,
                                       (float *)P.ptr(L.sB), hold ? nullptr : mean, P.ptr(L.sC),
                                       L.N, nullptr, step ? P.ptr(L.sProbs) : nullptr, L.N);
                if (rc == FG_OK && hold) {
                    ctx->mean_src = (const float *)P.ptr(L.sB);
                    ctx->mean_rows = L.M;
                    ctx->mean_dst = mean;
                }
                break;
            }
            case LK_ELT: {
                fg::EltProgram p;
                rc = elt_program(P, L, &p);
                if (rc == FG_OK) rc = fg::launch_eltwise(ctx, p);
                break;
            }
            case LK_FILL0:
                rc = fg_fill_u32(ctx, P.ptr(L.sC), 0u, L.count);
                break;
            default:
                fg::set_error("plan: unknown launch kind %d", L.kind);
                return FG_ERR_INTERNAL;
        }
        if (rc != FG_OK) return rc;
    }
    if (pending)
        if (int r = (*after_group)(group_end)) return r;
    ctx->defer_reduce = false;
    return FG_OK;
}

// The captured backward list.
const std::vector<Launch> &captured_bwd(const fg_plan &P) {
    return P.ce_fused_possible ? P.bwd_fused : P.bwd_seed;
}

// Byte ranges a launch reads or writes (its slots, whole).
std::vector<fg::ByteRange> launch_ranges(const fg_plan &P, const Launch &L) {
    std::vector<int> sl = {L.sA, L.sB, L.sC, L.sZ, L.sBias, L.sExtra, L.sProbs, L.label_slot};
    for (int k = 0; k < fg::kEltMaxSrc; ++k) sl.push_back(L.src_slot[k]);
    for (int k = 0; k < fg::kEltMaxDst; ++k) sl.push_back(L.dst_slot[k]);
    std::vector<fg::ByteRange> r;
    for (int x : sl)
        if (x != kNone && P.ptr(x)) {
            const uintptr_t b = (uintptr_t)P.ptr(x);
            r.push_back({b, b + P.slots[x].bytes});
        }
    return r;
}

// For each optimised input (in opt_inputs order): the index of the last
// launch of the last launch group of the captured backward that reads or
// writes its value or gradient (-1: none does).  A launch group is what
// run() launches together (a layer's dW and dX pair).  Needs bound inputs.
std::vector<int> adam_group_after(const fg_plan &P) {
    const std::vector<Launch> &bwd = captured_bwd(P);
    std::vector<std::vector<fg::ByteRange>> lr;
    for (const Launch &L : bwd) lr.push_back(launch_ranges(P, L));
    std::vector<int> after;
    for (uint32_t idx : P.opt_inputs) {
        const uint32_t n = P.inputs[idx];
        const uint64_t bytes = (uint64_t)P.shape[n].numel() * esize(P.dtype[n]);
        std::vector<fg::ByteRange> mine;
        for (const void *q : {P.ptr(P.input_slot[idx]), P.ptr(P.grad_slot[n])})
            mine.push_back({(uintptr_t)q, (uintptr_t)q + bytes});
        int last = -1;
        for (size_t i = 0; i < bwd.size(); ++i) {
            bool hit = false;
            for (const fg::ByteRange &a : lr[i])
                for (const fg::ByteRange &b : mine) hit = hit || a.overlaps(b);
            if (!hit) continue;
            // run() launches a pair (pair_next at i-1 or i) as one group.
            size_t end = i;
            if (bwd[i].pair_next && i + 1 < bwd.size()) end = i + 1;
            last = std::max(last, (int)end);
        }
        after.push_back(last);
    }
    return after;
}

int ensure_mt(fg_plan &P) {
    if (!P.mt_dirty) return FG_OK;
    for (uint32_t idx : P.opt_inputs)
        FG_REQUIRE(P.ptr(P.input_slot[idx]), FG_ERR_INVALID_ARGUMENT,
                   "dispatch_optim: input %u is not bound", idx);
    if (P.mt_all) fg_mt_destroy(P.mt_all);
    P.mt_all = nullptr;
    for (fg_mt *m : P.mt_single)
        if (m) fg_mt_destroy(m);
    P.mt_single.assign(P.inputs.size(), nullptr);
    if (P.opt_inputs.empty()) {
        P.mt_dirty = false;
        return FG_OK;
    }
    const bool adam = P.g.optim == FG_OPTIM_ADAM;
    std::vector<void *> pp, gg;
    std::vector<float *> mm, vv;
    std::vector<uint64_t> sz;
    std::vector<int> dts;
    for (uint32_t idx : P.opt_inputs) {
        const uint32_t n = P.inputs[idx];
        pp.push_back(P.ptr(P.input_slot[idx]));
        gg.push_back(P.ptr(P.grad_slot[n]));
        dts.push_back(P.dtype[n]);
        if (adam) {
            mm.push_back((float *)P.ptr(P.m_slot[idx]));
            vv.push_back((float *)P.ptr(P.v_slot[idx]));
        }
        sz.push_back((uint64_t)P.shape[n].numel());
    }
    int rc = fg_mt_create_x(P.ctx, (int)pp.size(), dts.data(), pp.data(), gg.data(),
                            adam ? mm.data() : nullptr, adam ? vv.data() : nullptr, sz.data(),
                            &P.mt_all);
    if (rc) return rc;
    for (size_t k = 0; k < P.opt_inputs.size(); ++k) {
        rc = fg_mt_create_x(P.ctx, 1, &dts[k], &pp[k], &gg[k], adam ? &mm[k] : nullptr,
                            adam ? &vv[k] : nullptr, &sz[k], &P.mt_single[P.opt_inputs[k]]);
        if (rc) return rc;
    }
    for (fg_mt *m : P.mt_groups)
        if (m) fg_mt_destroy(m);
    P.mt_groups.clear();
    P.mt_group_after.clear();
    // Only fp32 plans: the 16-bit GEMM tiles leave no room on a CU for the
    // update's workgroups beside them, which then wait for the GEMMs and
    // stretch the step (bf16 c5 step 2.05 -> 2.16 ms with a full grid per
    // group, 2.8-9.9 ms with 256 down to 32 workgroups).
    bool all_f32 = true;
    for (int d : dts) all_f32 = all_f32 && d == FG_DTYPE_F32;
    if (adam && all_f32) {
        // Captured steps: one tensor list per group of inputs the backward
        // releases together, in the order the backward releases them.
        std::map<int, std::vector<size_t>> by_after;
        const std::vector<int> after = adam_group_after(P);
        for (size_t k = 0; k < after.size(); ++k) by_after[after[k]].push_back(k);
        for (const auto &kv : by_after) {
            std::vector<void *> p2, g2;
            std::vector<float *> m2, v2;
            std::vector<uint64_t> s2;
            std::vector<int> d2;
            for (size_t k : kv.second) {
                p2.push_back(pp[k]);
                g2.push_back(gg[k]);
                m2.push_back(mm[k]);
                v2.push_back(vv[k]);
                s2.push_back(sz[k]);
                d2.push_back(dts[k]);
            }
            fg_mt *m = nullptr;
            rc = fg_mt_create_x(P.ctx, (int)p2.size(), d2.data(), p2.data(), g2.data(), m2.data(),
                                v2.data(), s2.data(), &m);
            if (rc) return rc;
            P.mt_groups.push_back(m);
            P.mt_group_after.push_back(kv.first);
        }
        if (!P.side) {
            hipError_t e = hipStreamCreateWithFlags(&P.side, hipStreamNonBlocking);
            if (e != hipSuccess) return fg::hip_fail(e, "hipStreamCreateWithFlags", __FILE__, __LINE__);
        }
        while (P.events.size() < P.mt_groups.size() + 2) {
            hipEvent_t ev = nullptr;
            hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
            if (e != hipSuccess) return fg::hip_fail(e, "hipEventCreateWithFlags", __FILE__, __LINE__);
            P.events.push_back(ev);
        }
    }
    P.mt_dirty = false;
    return FG_OK;
}

// The backward of a captured Adam step with the optimiser's update in
// groups (ensure_mt): the step counter advances on the main stream first;
// each group's update goes to the second stream once the main stream has
// run the launch group that last touches its tensors (an event recorded
// there and waited for on the second stream), so the bandwidth-bound
// updates overlap the remaining GEMMs.  The second stream rejoins the main
// one at the end.  Every parameter gets exactly the update of the single
// multi-tensor launch (same kernel, same operations per element).
// Workgroups of each grouped update (each walks several 1024-element
// chunks): few enough to sit beside the GEMM's tiles rather than queue
// ahead of them.  c5 fp32 step: 10.02-10.03 ms with the single update at
// the end; 9.86-9.90 with 256 or 512 workgroups per group; 9.98-10.01 with
// 1024; 10.2 / 11.0 / 13.0 ms with 128 / 64 / 32 (too slow to finish
// within the backward).  Since the pair launches raise their waves' issue
// priority over the update (k_gemm_pair.hip), larger grids finish the
// updates sooner at less cost to the pairs: 512 workgroups per group, and
// 1024 for the update beside the final launch, whose end the step waits for:
// 9.607 ms per c5 step, against 9.624 with 512 for every group and 9.650
// with 256 (1024 beside the last two launches), three passes on one box.
#ifndef FG_SIDE_ADAM_BLOCKS  // knobs for measurement builds
#define FG_SIDE_ADAM_BLOCKS 512
#endif
#ifndef FG_SIDE_ADAM_FINAL_BLOCKS
#define FG_SIDE_ADAM_FINAL_BLOCKS 1024
#endif
constexpr uint32_t kSideAdamBlocks = FG_SIDE_ADAM_BLOCKS;
constexpr uint32_t kSideAdamFinalBlocks = FG_SIDE_ADAM_FINAL_BLOCKS;
int run_bwd_adam_overlapped(fg_plan &P, const std::vector<Launch> &bwd) {
    fg_ctx *ctx = &P.wctx;
    const size_t G = P.mt_groups.size();
    bool forked = false;  // the second stream has joined the capture
    // The second stream starts from the loss: it runs the mean loss the loss
    // launch held (ctx->mean_dst) and the step counter's advance, both off
    // the backward's path, before the first group's update (c5 step 9.608 ->
    // 9.600 ms, three passes on one box).  Its first node is created after
    // the backward's first launch, which so keeps the main stream's queue.
    FG_HIP(hipEventRecord(P.events[G + 1], ctx->stream));
    bool side_head = true;  // that first work not issued yet
    // The main stream records group g's event once it has run the launch
    // group that releases g; the update itself is issued one launch group
    // later, after the main stream's next launch.  The dependencies are the
    // same either way, but a replayed graph runs a node's first-created child
    // on the node's hardware queue: created first, the next GEMM keeps the
    // backward on one queue, and the updates branch off onto another (created
    // first, an update took the queue and a later GEMM queued behind one,
    // ~120 us per c5 step).
    std::vector<size_t> pending;
    auto mark = [&](size_t g) -> int {
        FG_HIP(hipEventRecord(P.events[g], ctx->stream));
        pending.push_back(g);
        return FG_OK;
    };
    auto issue = [&](bool last, bool beside_final = false) -> int {
        if (side_head) {
            side_head = false;
            FG_HIP(hipStreamWaitEvent(P.side, P.events[G + 1], 0));
            forked = true;
            if (ctx->mean_dst) {
                if (int r = fg::launch_mean_loss(P.side, ctx->mean_src, ctx->mean_rows,
                                                 ctx->mean_dst))
                    return r;
                ctx->mean_dst = nullptr;
            }
            if (int r = fg::adam_dev_advance_on(P.side, P.lr, P.b1, P.b2, P.ptr(P.adam_slot)))
                return r;
        }
        for (size_t g : pending) {
            FG_HIP(hipStreamWaitEvent(P.side, P.events[g], 0));
            forked = true;
            // Nothing runs beside the backward's last updates: a full grid.
            if (int r = fg::mt_adam_dev_update(P.mt_groups[g], P.side, P.b1, P.b2, P.eps,
                                               P.ptr(P.adam_slot), 0,
                                               last           ? 0u
                                               : beside_final ? kSideAdamFinalBlocks
                                                              : kSideAdamBlocks))
                return r;
        }
        pending.clear();
        return FG_OK;
    };
    int rc = FG_OK;
    for (size_t g = 0; g < G && rc == FG_OK; ++g)  // inputs the backward never touches
        if (P.mt_group_after[g] < 0) rc = mark(g);
    const std::function<int(size_t)> after = [&](size_t last) -> int {
        // Called after the final launch group too (last = bwd.size() - 1):
        // the updates issued then run beside that final launch.
        if (int r = issue(false, last + 1 >= bwd.size())) return r;
        for (size_t g = 0; g < G; ++g)
            if (P.mt_group_after[g] == (int)last)
                if (int r = mark(g)) return r;
        return FG_OK;
    };
    if (rc == FG_OK) rc = run(P, bwd, false, false, nullptr, nullptr, nullptr, -1, &after);
    if (rc == FG_OK) rc = issue(true);
    // Rejoin whatever happened, so the capture can end.
    if (forked) {
        const hipError_t e1 = hipEventRecord(P.events[G], P.side);
        const hipError_t e2 = hipStreamWaitEvent(ctx->stream, P.events[G], 0);
        if (rc == FG_OK && e1 != hipSuccess)
            return fg::hip_fail(e1, "hipEventRecord", __FILE__, __LINE__);
        if (rc == FG_OK && e2 != hipSuccess)
            return fg::hip_fail(e2, "hipStreamWaitEvent", __FILE__, __LINE__);
    }
    return rc;
}

// The memory the optimiser touches: every optimised input and its gradient.
std::vector<fg::ByteRange> optim_ranges(const fg_plan &P) {
    std::vector<fg::ByteRange> r;
    for (uint32_t idx : P.opt_inputs) {
        const uint32_t n = P.inputs[idx];
        const uint64_t bytes = (uint64_t)P.shape[n].numel() * esize(P.dtype[n]);
        for (const void *q : {P.ptr(P.input_slot[idx]), P.ptr(P.grad_slot[n])})
            r.push_back({(uintptr_t)q, (uintptr_t)q + bytes});
    }
    return r;
}

int run_optim(fg_plan &P, fg_mt *mt) {
    // Work held for this launch (captured steps): the backward's last
    // summing pass, beside SGD when the two touch disjoint memory, else
    // first; the mean loss of a loss finished in the head GEMM, beside SGD
    // (it touches only the loss buffers), else first.
    const bool sgd = mt && P.g.optim == FG_OPTIM_SGD;
    if (P.wctx.pending_splits > 0) {
        bool fuse = sgd;
        if (fuse) {
            fg::ByteRange red[3];
            fg::pending_reduce_ranges(&P.wctx, red);
            for (const fg::ByteRange &o : optim_ranges(P))
                for (const fg::ByteRange &q : red) fuse = fuse && !q.overlaps(o);
        }
        if (!fuse)
            if (int rc = fg::launch_pending_reduce(&P.wctx)) return rc;
    }
    if (P.wctx.pending_splits > 0 || P.wctx.mean_dst) {
        if (sgd) return fg::sgd_step_with_pending(P.ctx, mt, P.lr, 1, &P.wctx);
        if (int rc = fg::launch_pending_mean(&P.wctx)) return rc;
    }
    if (!mt) return FG_OK;
    if (P.g.optim == FG_OPTIM_ADAM)
        return fg::mt_adam_dev(P.ctx, mt, P.lr, P.b1, P.b2, P.eps, P.ptr(P.adam_slot), 0);
    // SGD zeroes the gradient after the update (basic_optim.rs:27-28).
    return fg_sgd_step(P.ctx, mt, P.lr, 1);
}

void drop_graph(fg_plan &P) {
    if (P.exec) (void)hipGraphExecDestroy(P.exec);
    if (P.graph) (void)hipGraphDestroy(P.graph);
    P.exec = nullptr;
    P.graph = nullptr;
}

}  // namespace

// ====================================================================== ABI
FG_API int fg_memcpy_h2d(fg_ctx *ctx, void *d_dst, const void *src, uint64_t bytes) {
    FG_REQUIRE(ctx && (bytes == 0 || (d_dst && src)), FG_ERR_INVALID_ARGUMENT,
               "fg_memcpy_h2d: NULL argument");
    if (!bytes) return FG_OK;
    FG_HIP(hipMemcpyAsync(d_dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    FG_HIP(hipStreamSynchronize(ctx->stream));
    return FG_OK;
}

FG_API int fg_memcpy_d2h(fg_ctx *ctx, void *dst, const void *d_src, uint64_t bytes) {
    FG_REQUIRE(ctx && (bytes == 0 || (dst && d_src)), FG_ERR_INVALID_ARGUMENT,
               "fg_memcpy_d2h: NULL argument");
    if (!bytes) return FG_OK;
    FG_HIP(hipMemcpyAsync(dst, d_src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    FG_HIP(hipStreamSynchronize(ctx->stream));
    return FG_OK;
}

FG_API int fg_graph_create(int loss, int optim, fg_graph **out) {
    FG_REQUIRE(out, FG_ERR_INVALID_ARGUMENT, "fg_graph_create: out is NULL");
    FG_REQUIRE(loss >= FG_LOSS_MSE && loss <= FG_LOSS_CE, FG_ERR_INVALID_ARGUMENT,
               "fg_graph_create: unknown loss %d", loss);
    FG_REQUIRE(optim == FG_OPTIM_SGD || optim == FG_OPTIM_ADAM, FG_ERR_INVALID_ARGUMENT,
               "fg_graph_create: unknown optimiser %d", optim);
    fg_graph *g = new fg_graph;
    g->loss = loss;
    g->optim = optim;
    *out = g;
    return FG_OK;
}

FG_API int fg_graph_destroy(fg_graph *g) {
    delete g;
    return FG_OK;
}

FG_API int fg_graph_new_field(fg_graph *g, uint32_t *field) {
    FG_REQUIRE(g && field, FG_ERR_INVALID_ARGUMENT, "fg_graph_new_field: NULL argument");
    *field = ++g->nfields;
    return FG_OK;
}

FG_API int fg_graph_input(fg_graph *g, const uint32_t *fields, int rank, uint32_t *node) {
    FG_REQUIRE(g && node && (fields || rank == 0), FG_ERR_INVALID_ARGUMENT,
               "fg_graph_input: NULL argument");
    FG_REQUIRE(rank >= 1 && rank <= 8, FG_ERR_GRAPH, "fg_graph_input: rank %d not in [1, 8]",
               rank);
    for (int d = 0; d < rank; ++d)
        FG_REQUIRE(fields[d] >= 1 && fields[d] <= g->nfields, FG_ERR_GRAPH,
                   "fg_graph_input: field %u was not declared", fields[d]);
    GNode nd;
    nd.op = FG_OP_INPUT;
    nd.fields.assign(fields, fields + rank);
    g->nodes.push_back(nd);
    *node = (uint32_t)g->nodes.size() - 1;
    return FG_OK;
}

FG_API int fg_graph_input_x(fg_graph *g, const uint32_t *fields, int rank, int dtype,
                           uint32_t *node) {
    FG_REQUIRE(dtype >= FG_DTYPE_F32 && dtype <= FG_DTYPE_BF16, FG_ERR_UNSUPPORTED,
               "fg_graph_input_x: element type %d is not F32 / F16 / BF16", dtype);
    int rc = fg_graph_input(g, fields, rank, node);
    if (rc == FG_OK) g->nodes[*node].dtype = dtype;
    return rc;
}

FG_API int fg_graph_constant(fg_graph *g, int dtype, float value, uint32_t *node) {
    FG_REQUIRE(dtype >= FG_DTYPE_F32 && dtype <= FG_DTYPE_BF16, FG_ERR_UNSUPPORTED,
               "fg_graph_constant: element type %d is not F32 / F16 / BF16", dtype);
    int rc = fg_graph_constant_f32(g, round_host(dtype, value), node);
    if (rc == FG_OK) g->nodes[*node].dtype = dtype;
    return rc;
}

FG_API int fg_graph_constant_f32(fg_graph *g, float value, uint32_t *node) {
    FG_REQUIRE(g && node, FG_ERR_INVALID_ARGUMENT, "fg_graph_constant_f32: NULL argument");
    GNode nd;
    nd.op = FG_OP_CONST;
    nd.value = value;
    g->nodes.push_back(nd);
    *node = (uint32_t)g->nodes.size() - 1;
    return FG_OK;
}

FG_API int fg_graph_op(fg_graph *g, int op, const uint32_t *inputs, int n_inputs, uint32_t *node) {
    FG_REQUIRE(g && node && (inputs || n_inputs == 0), FG_ERR_INVALID_ARGUMENT,
               "fg_graph_op: NULL argument");
    FG_REQUIRE(op != FG_OP_INPUT && op != FG_OP_CONST, FG_ERR_INVALID_ARGUMENT,
               "fg_graph_op: op %d is a leaf (use fg_graph_input / fg_graph_constant)", op);
    // A GraphOp::Custom the mirror could not map to a ferrograd-nn builder
    // (backend/mod.rs:659-726) arrives as a code outside fg_op.
    FG_REQUIRE(op >= FG_OP_ADD && op <= FG_OP_BIAS_ADD, FG_ERR_UNSUPPORTED,
               "fg_graph_op: operation kind %d is not one this backend lowers (fg_op covers "
               "ferrograd-nn's builders: add sub mul div matmul relu gelu elu tanh exp log abs "
               "neg softmax bias_add)", op);
    FG_REQUIRE(n_inputs == arity(op), FG_ERR_GRAPH, "fg_graph_op: %s takes %d inputs, got %d",
               op_name(op), arity(op), n_inputs);
    for (int k = 0; k < n_inputs; ++k)
        FG_REQUIRE(inputs[k] < g->nodes.size(), FG_ERR_GRAPH,
                   "fg_graph_op: input node %u does not exist", inputs[k]);
    GNode nd;
    nd.op = op;
    nd.in.assign(inputs, inputs + n_inputs);
    g->nodes.push_back(nd);
    *node = (uint32_t)g->nodes.size() - 1;
    return FG_OK;
}

FG_API int fg_graph_set_input_flags(fg_graph *g, uint32_t node, uint32_t flags) {
    FG_REQUIRE(g && node < g->nodes.size() && g->nodes[node].op == FG_OP_INPUT,
               FG_ERR_INVALID_ARGUMENT, "fg_graph_set_input_flags: node %u is not an input", node);
    g->nodes[node].flags = flags;
    return FG_OK;
}

FG_API int fg_graph_num_nodes(const fg_graph *g, uint32_t *n) {
    FG_REQUIRE(g && n, FG_ERR_INVALID_ARGUMENT, "fg_graph_num_nodes: NULL argument");
    *n = (uint32_t)g->nodes.size();
    return FG_OK;
}

FG_API int fg_graph_validate(const fg_graph *g, const uint32_t *meta, int n_meta) {
    FG_REQUIRE(g && (meta || n_meta == 0), FG_ERR_INVALID_ARGUMENT,
               "fg_graph_validate: NULL argument");
    std::vector<Shape> sh;
    return infer_shapes(*g, meta, n_meta, sh);
}

FG_API int fg_plan_create(fg_ctx *ctx, const fg_graph *g, const uint32_t *meta, int n_meta,
                          fg_plan **out) {
    FG_REQUIRE(g && out && meta, FG_ERR_INVALID_ARGUMENT, "fg_plan_create: NULL argument");
    std::unique_ptr<fg_plan> P(new fg_plan);
    P->ctx = ctx;
    P->g = *g;
    P->meta.assign(meta, meta + n_meta);
    int rc = infer_shapes(P->g, meta, n_meta, P->shape);
    if (rc) return rc;
    const fg_graph &G = P->g;
    const size_t nn = G.nodes.size();
    P->last = (int)nn - 1;
    // Element types: an operation takes its first input's type
    // (op/binary.rs:232, unary.rs, matmul/mod.rs:294).
    P->dtype.assign(nn, FG_DTYPE_F32);
    for (uint32_t i = 0; i < nn; ++i) {
        const GNode &nd = G.nodes[i];
        P->dtype[i] = nd.in.empty() ? nd.dtype : P->dtype[nd.in[0]];
    }
    float lr;
    std::memcpy(&lr, &meta[0], 4);
    P->lr = lr;
    P->users.assign(nn, {});
    for (uint32_t i = 0; i < nn; ++i)
        for (uint32_t x : G.nodes[i].in) P->users[x].push_back(i);
    compute_saved(G, P->users, P->save);
    // needs_grad: depends on an input that takes a gradient.
    P->needs_grad.assign(nn, 0);
    for (uint32_t i = 0; i < nn; ++i) {
        const GNode &nd = G.nodes[i];
        if (nd.op == FG_OP_INPUT) {
            P->needs_grad[i] = !(nd.flags & FG_INPUT_NO_GRAD);
            P->inputs.push_back(i);
        } else if (nd.op != FG_OP_CONST) {
            for (uint32_t x : nd.in) P->needs_grad[i] |= P->needs_grad[x];
        }
    }
    // Products with a row-broadcast vector that needs a gradient would need
    // a reduction of a product: not supported.
    for (uint32_t i = 0; i < nn; ++i) {
        const GNode &nd = G.nodes[i];
        if (nd.op != FG_OP_MUL && nd.op != FG_OP_DIV) continue;
        for (uint32_t x : nd.in) {
            const Shape &sx = P->shape[x];
            FG_REQUIRE(sx.scalar || sx.numel() == P->shape[i].numel() || !P->needs_grad[x],
                       FG_ERR_UNSUPPORTED,
                       "%s %u: gradient of a row-broadcast operand is not supported",
                       op_name(nd.op), i);
        }
    }
    P->ce_fused_possible = G.loss == FG_LOSS_CE && G.nodes.back().op == FG_OP_SOFTMAX;

    // GEMM groups.
    P->group_of.assign(nn, kNone);
    for (uint32_t i = 0; i < nn; ++i) {
        if (G.nodes[i].op != FG_OP_MATMUL) continue;
        FG_REQUIRE(P->dtype[G.nodes[i].in[0]] == P->dtype[G.nodes[i].in[1]], FG_ERR_UNSUPPORTED,
                   "matmul %u: operands of different element types (%s, %s)", i,
                   dtype_name(P->dtype[G.nodes[i].in[0]]), dtype_name(P->dtype[G.nodes[i].in[1]]));
        Group gr;
        gr.mm = (int)i;
        int cur = (int)i;
        if (P->users[i].size() == 1) {
            const uint32_t u = P->users[i][0];
            const GNode &un = G.nodes[u];
            if ((un.op == FG_OP_BIAS_ADD || un.op == FG_OP_ADD) && un.in[0] == i &&
                un.in[1] != i) {
                const Shape &sb = P->shape[un.in[1]];
                if (sb.vector && sb.cols == P->shape[i].cols &&
                    G.nodes[un.in[1]].op != FG_OP_CONST && P->dtype[un.in[1]] == P->dtype[i]) {
                    gr.bias_node = (int)u;
                    gr.bias_src = (int)un.in[1];
                    cur = (int)u;
                }
            }
        }
        gr.pre = cur;
        if (P->users[cur].size() == 1) {
            const uint32_t u = P->users[cur][0];
            const int op = G.nodes[u].op;
            if ((op == FG_OP_RELU || op == FG_OP_GELU) && G.nodes[u].in[0] == (uint32_t)cur)
                gr.act_node = (int)u;
        }
        gr.fin = gr.act_node != kNone ? gr.act_node : cur;
        const int gi = (int)P->groups.size();
        P->groups.push_back(gr);
        P->group_of[gr.mm] = gi;
        if (gr.bias_node != kNone) P->group_of[gr.bias_node] = gi;
        if (gr.act_node != kNone) P->group_of[gr.act_node] = gi;
    }

    // Slots.
    P->val_slot.assign(nn, kNone);
    P->grad_slot.assign(nn, kNone);
    P->input_slot.assign(P->inputs.size(), kNone);
    for (size_t k = 0; k < P->inputs.size(); ++k) {
        const uint32_t n = P->inputs[k];
        P->input_slot[k] = P->new_external((uint64_t)P->shape[n].numel(), P->dtype[n]);
        P->val_slot[n] = P->input_slot[k];
    }
    for (uint32_t i = 0; i < nn; ++i) {
        const int op = G.nodes[i].op;
        if (op == FG_OP_INPUT || op == FG_OP_CONST) continue;
        P->val_slot[i] = P->new_slot((uint64_t)P->shape[i].numel(), P->dtype[i]);
    }
    for (const Group &gr : P->groups)  // the pre-bias product is not materialised
        if (gr.bias_node != kNone) P->val_slot[gr.mm] = P->val_slot[gr.bias_node];
    for (uint32_t i = 0; i < nn; ++i) {
        if (G.nodes[i].op == FG_OP_CONST) continue;
        if (P->needs_grad[i] || (int)i == P->last)
            P->grad_slot[i] = P->new_slot((uint64_t)P->shape[i].numel(), P->dtype[i]);
    }
    for (const Group &gr : P->groups)  // d(matmul) == d(bias add)
        if (gr.bias_node != kNone && P->grad_slot[gr.bias_node] != kNone)
            P->grad_slot[gr.mm] = P->grad_slot[gr.bias_node];
    const Shape &ls = P->shape[P->last];
    // Loss and target: CE on a final softmax keeps fp32 per-row losses and
    // u32 labels; otherwise both are of the output's type (dispatch/mod.rs:
    // 551-562 sizes loss_t by the last node's type).
    const int ldt = P->dtype[P->last];
    if (G.loss == FG_LOSS_CE) {
        P->target_bytes = (uint64_t)ls.rows * 4;
        P->target_slot = P->new_external((uint64_t)ls.rows);
        P->loss_slot = P->ce_fused_possible ? P->new_slot((uint64_t)ls.rows)
                                            : P->new_slot((uint64_t)ls.numel(), ldt);
    } else {
        P->target_bytes = (uint64_t)ls.numel() * esize(ldt);
        P->target_slot = P->new_external((uint64_t)ls.numel(), ldt);
        P->loss_slot = P->new_slot((uint64_t)ls.numel(), ldt);
    }
    P->mean_slot = P->new_slot(1);
    // Optimiser.
    for (size_t k = 0; k < P->inputs.size(); ++k) {
        const GNode &nd = G.nodes[P->inputs[k]];
        if (!(nd.flags & (FG_INPUT_NO_GRAD | FG_INPUT_FROZEN))) P->opt_inputs.push_back((uint32_t)k);
    }
    P->m_slot.assign(P->inputs.size(), kNone);
    P->v_slot.assign(P->inputs.size(), kNone);
    if (G.optim == FG_OPTIM_ADAM) {
        for (uint32_t k : P->opt_inputs) {
            const uint64_t e = (uint64_t)P->shape[P->inputs[k]].numel();
            P->m_slot[k] = P->new_slot(e);  // fp32 state whatever the parameter type
            P->v_slot[k] = P->new_slot(e);
        }
        P->adam_slot = P->new_slot((fg::adam_dev_state_bytes() + 3) / 4);
    }
    // Exposed lists in SaveIndicator order.
    for (uint32_t i = 0; i < nn; ++i) {
        if (P->save[i] & kDefFwd) P->saved_nodes.push_back(i);
        if ((P->save[i] & kDefBwd) && P->grad_slot[i] != kNone) P->grad_nodes.push_back(i);
    }

    // Lowering (launches refer to slots; lowering may add temporaries).
    if ((rc = lower_forward(*P))) return rc;
    if ((rc = lower_loss(*P))) return rc;
    if ((rc = lower_backward(*P, false, P->bwd_seed))) return rc;
    if (P->ce_fused_possible && (rc = lower_backward(*P, true, P->bwd_fused))) return rc;

    // Static bounds check of every launch against the sizes of the slots it
    // touches, so a planner slip is an error here rather than a device fault.
    for (auto *list : {&P->fwd, &P->loss, &P->bwd_seed, &P->bwd_fused})
        for (const Launch &L : *list)
            if ((rc = check_launch(*P, L))) return rc;

    // Workspace: at least 1 MiB (what lets few-tile fp32 GEMMs split K), the
    // partial sums of the largest unfused bias-gradient reduction, and the K
    // slices of the largest split 16-bit GEMM (fp32 slots of its output: the
    // 1000-wide head of a batch-2048 MLP takes 4 x 8 MB).
    {
        const int cus = ctx && ctx->cu_count > 0 ? ctx->cu_count : 256;
        uint64_t ws = 1u << 20;
        for (auto *list : {&P->bwd_seed, &P->bwd_fused})
            for (const Launch &L : *list)
                if (L.kind == LK_BIAS_GRAD)
                    ws = std::max<uint64_t>(ws, fg::bias_grad_ws_bytes(cus, L.M, L.N));
        for (auto *list : {&P->fwd, &P->bwd_seed, &P->bwd_fused})
            for (const Launch &L : *list)
                if ((L.kind == LK_GEMM || L.kind == LK_GEMM_BWD) && L.dtype != FG_DTYPE_F32) {
                    const bool cs = L.kind == LK_GEMM && L.sExtra != kNone;  // dW + dbias (TN)
                    ws = std::max<uint64_t>(ws, fg::gemm16_split_ws_bytes(
                                                    cus, cs ? FG_TN : L.layout, L.M, L.N, L.K, cs));
                }
        P->ws_bytes = ws;
        P->ws_slot = P->new_slot(ws / 4);
    }

    // Arena: every plan-owned tensor in one allocation, each starting 4 KiB
    // x (1 + k mod 15) past a 64 KiB boundary (k: the slot's place in the
    // arena).  The streams an HBM-bound kernel walks in step (a parameter's
    // gradient, Adam m and v; a layer's node values) then start on different
    // DRAM banks rather than on the same one: 3 + 3 and 4 + 3 streams ran
    // 5-10 % faster staggered by 4 KiB than at equal alignment.  No slot
    // starts on a 64 KiB boundary, where large caller buffers (parameters,
    // inputs) lie.  The padding costs under 64 KiB per slot.
    uint64_t off = 0;
    int k = 0;
    for (Slot &s : P->slots) {
        if (s.external) continue;
        constexpr uint64_t kWin = 64 * 1024, kStep = 4 * 1024;
        const uint64_t want = kStep * (1 + (uint64_t)(k++ % 15));
        off += (want + kWin - off % kWin) % kWin;
        s.offset = off;
        off += (s.bytes + 255) & ~uint64_t(255);
    }
    P->arena_bytes = off;
    if (!ctx) {  // dry plan: lowering only (describe), nothing allocated
        *out = P.release();
        return FG_OK;
    }
    FG_HIP(hipSetDevice(ctx->device));
    if (off) {
        hipError_t e = hipMalloc((void **)&P->arena, off);
        if (e != hipSuccess)
            return fg::hip_fail(e, "fg_plan_create: arena hipMalloc", __FILE__, __LINE__);
        // Zero the arena once (grads of unreached inputs, optimiser state,
        // the Adam step counter) with a fill kernel.
        rc = fg_fill_u32(ctx, P->arena, 0u, off / 4);
        if (rc) return rc;
    }
    P->wctx.device = ctx->device;
    P->wctx.stream = ctx->stream;
    P->wctx.own_stream = false;
    P->wctx.cu_count = ctx->cu_count;
    std::memcpy(P->wctx.arch, ctx->arch, sizeof ctx->arch);
    P->wctx.ws = P->ptr(P->ws_slot);
    P->wctx.ws_bytes = P->ws_bytes;
    P->wctx.ws_fixed = true;
    FG_HIP(hipStreamSynchronize(ctx->stream));
    *out = P.release();
    return FG_OK;
}

FG_API int fg_plan_destroy(fg_plan *p) {
    if (!p) return FG_OK;
    if (p->ctx) {
        (void)hipSetDevice(p->ctx->device);
        (void)hipStreamSynchronize(p->ctx->stream);
    }
    delete p;
    return FG_OK;
}

FG_API int fg_plan_count(const fg_plan *p, int role, int *count) {
    FG_REQUIRE(p && count, FG_ERR_INVALID_ARGUMENT, "fg_plan_count: NULL argument");
    switch (role) {
        case FG_ROLE_FORWARD_OUT: case FG_ROLE_SEED: case FG_ROLE_LOSS: case FG_ROLE_TARGET:
            *count = 1;
            break;
        case FG_ROLE_MEAN_LOSS: *count = p->ce_fused_possible ? 1 : 0; break;
        case FG_ROLE_FORWARD_SAVED: *count = (int)p->saved_nodes.size(); break;
        case FG_ROLE_GRAD: *count = (int)p->grad_nodes.size(); break;
        case FG_ROLE_INPUT: *count = (int)p->inputs.size(); break;
        case FG_ROLE_STATE:
            *count = p->g.optim == FG_OPTIM_ADAM ? 2 * (int)p->opt_inputs.size() : 0;
            break;
        default:
            fg::set_error("fg_plan_count: unknown role %d", role);
            return FG_ERR_INVALID_ARGUMENT;
    }
    return FG_OK;
}

namespace {
int plan_slot_of(const fg_plan *p, int role, int index, int *slot_out, uint32_t *node_out);
}

FG_API int fg_plan_tensor(const fg_plan *p, int role, int index, void **d_ptr, uint64_t *bytes,
                          uint32_t *node) {
    int slot = kNone;
    uint32_t nd = 0;
    int rc = plan_slot_of(p, role, index, &slot, &nd);
    if (rc) return rc;
    if (d_ptr) *d_ptr = p->ptr(slot);
    if (bytes) *bytes = p->slots[slot].used;
    if (node) *node = nd;
    return FG_OK;
}

FG_API int fg_plan_tensor_dtype(const fg_plan *p, int role, int index, int *dtype) {
    FG_REQUIRE(dtype, FG_ERR_INVALID_ARGUMENT, "fg_plan_tensor_dtype: dtype is NULL");
    int slot = kNone;
    uint32_t nd = 0;
    int rc = plan_slot_of(p, role, index, &slot, &nd);
    if (rc) return rc;
    *dtype = p->slots[slot].dtype;
    return FG_OK;
}

namespace {
int plan_slot_of(const fg_plan *p, int role, int index, int *slot_out, uint32_t *node_out) {
    FG_REQUIRE(p, FG_ERR_INVALID_ARGUMENT, "fg_plan_tensor: plan is NULL");
    int cnt = 0;
    int rc = fg_plan_count(p, role, &cnt);
    if (rc) return rc;
    FG_REQUIRE(index >= 0 && index < cnt, FG_ERR_OUT_OF_BOUNDS,
               "fg_plan_tensor: index %d out of range for role %d (%d tensors)", index, role, cnt);
    int slot = kNone;
    uint32_t nd = 0;
    switch (role) {
        case FG_ROLE_FORWARD_OUT: nd = p->last; slot = p->val_slot[nd]; break;
        case FG_ROLE_SEED: nd = p->last; slot = p->grad_slot[nd]; break;
        case FG_ROLE_LOSS: nd = p->last; slot = p->loss_slot; break;
        case FG_ROLE_MEAN_LOSS: nd = p->last; slot = p->mean_slot; break;
        case FG_ROLE_TARGET: nd = p->last; slot = p->target_slot; break;
        case FG_ROLE_FORWARD_SAVED: nd = p->saved_nodes[index]; slot = p->val_slot[nd]; break;
        case FG_ROLE_GRAD: nd = p->grad_nodes[index]; slot = p->grad_slot[nd]; break;
        case FG_ROLE_INPUT: nd = p->inputs[index]; slot = p->input_slot[index]; break;
        case FG_ROLE_STATE: {
            const uint32_t k = p->opt_inputs[index / 2];
            nd = p->inputs[k];
            slot = (index % 2) ? p->v_slot[k] : p->m_slot[k];
            break;
        }
    }
    *slot_out = slot;
    *node_out = nd;
    return FG_OK;
}
}  // namespace

FG_API int fg_plan_bind_input(fg_plan *p, int index, void *d_ptr, uint64_t bytes) {
    FG_REQUIRE(p && d_ptr, FG_ERR_INVALID_ARGUMENT, "fg_plan_bind_input: NULL argument");
    FG_REQUIRE(index >= 0 && index < (int)p->inputs.size(), FG_ERR_OUT_OF_BOUNDS,
               "fg_plan_bind_input: input %d out of range (%zu inputs)", index, p->inputs.size());
    Slot &s = p->slots[p->input_slot[index]];
    FG_REQUIRE(bytes >= s.used, FG_ERR_SHAPE,
               "fg_plan_bind_input: input %d needs %llu bytes, got %llu", index,
               (unsigned long long)s.bytes, (unsigned long long)bytes);
    if (s.ext != d_ptr) {
        s.ext = d_ptr;
        p->mt_dirty = true;
        drop_graph(*p);
    }
    return FG_OK;
}

FG_API int fg_plan_bind_target(fg_plan *p, const void *d_ptr, uint64_t bytes) {
    FG_REQUIRE(p && d_ptr, FG_ERR_INVALID_ARGUMENT, "fg_plan_bind_target: NULL argument");
    Slot &s = p->slots[p->target_slot];
    FG_REQUIRE(bytes >= s.bytes, FG_ERR_SHAPE,
               "fg_plan_bind_target: target needs %llu bytes, got %llu",
               (unsigned long long)s.bytes, (unsigned long long)bytes);
    if (s.ext != d_ptr) {
        s.ext = const_cast<void *>(d_ptr);
        drop_graph(*p);
    }
    return FG_OK;
}

FG_API int fg_plan_set_lr(fg_plan *p, float lr) {
    FG_REQUIRE(p, FG_ERR_INVALID_ARGUMENT, "fg_plan_set_lr: plan is NULL");
    if (p->lr != lr) drop_graph(*p);
    p->lr = lr;
    return FG_OK;
}

FG_API int fg_plan_set_adam(fg_plan *p, float b1, float b2, float eps) {
    FG_REQUIRE(p, FG_ERR_INVALID_ARGUMENT, "fg_plan_set_adam: plan is NULL");
    FG_REQUIRE(b1 >= 0.f && b1 < 1.f && b2 >= 0.f && b2 < 1.f && eps >= 0.f,
               FG_ERR_INVALID_ARGUMENT, "fg_plan_set_adam: bad hyper-parameters");
    drop_graph(*p);
    p->b1 = b1;
    p->b2 = b2;
    p->eps = eps;
    return FG_OK;
}

FG_API int fg_plan_forward(fg_plan *p) {
    FG_REQUIRE(p && p->ctx, FG_ERR_INVALID_ARGUMENT, "fg_plan_forward: plan is NULL or has no device (dry plan)");
    FG_HIP(hipSetDevice(p->ctx->device));
    for (size_t k = 0; k < p->inputs.size(); ++k)
        FG_REQUIRE(p->ptr(p->input_slot[k]), FG_ERR_INVALID_ARGUMENT,
                   "dispatch_forward: input %zu is not bound", k);
    return run(*p, p->fwd);
}

FG_API int fg_plan_loss(fg_plan *p) {
    FG_REQUIRE(p && p->ctx, FG_ERR_INVALID_ARGUMENT, "fg_plan_loss: plan is NULL or has no device (dry plan)");
    FG_REQUIRE(p->ptr(p->target_slot), FG_ERR_INVALID_ARGUMENT,
               "dispatch_loss: no target bound (fg_plan_bind_target)");
    FG_HIP(hipSetDevice(p->ctx->device));
    int rc = run(*p, p->loss);
    if (rc == FG_OK && p->ce_fused_possible) p->ce_fused_pending = true;
    return rc;
}

FG_API int fg_plan_backward(fg_plan *p) {
    FG_REQUIRE(p && p->ctx, FG_ERR_INVALID_ARGUMENT, "fg_plan_backward: plan is NULL or has no device (dry plan)");
    FG_HIP(hipSetDevice(p->ctx->device));
    const bool fused = p->ce_fused_pending;
    p->ce_fused_pending = false;
    return run(*p, fused ? p->bwd_fused : p->bwd_seed);
}

FG_API int fg_plan_optim(fg_plan *p) {
    FG_REQUIRE(p && p->ctx, FG_ERR_INVALID_ARGUMENT, "fg_plan_optim: plan is NULL or has no device (dry plan)");
    FG_HIP(hipSetDevice(p->ctx->device));
    int rc = ensure_mt(*p);
    if (rc) return rc;
    return run_optim(*p, p->mt_all);
}

FG_API int fg_plan_single_optim(fg_plan *p, int input_index) {
    FG_REQUIRE(p && p->ctx, FG_ERR_INVALID_ARGUMENT, "fg_plan_single_optim: plan is NULL or has no device (dry plan)");
    FG_REQUIRE(input_index >= 0 && input_index < (int)p->inputs.size(), FG_ERR_OUT_OF_BOUNDS,
               "fg_plan_single_optim: input %d out of range", input_index);
    FG_HIP(hipSetDevice(p->ctx->device));
    int rc = ensure_mt(*p);
    if (rc) return rc;
    FG_REQUIRE(p->g.optim != FG_OPTIM_ADAM, FG_ERR_UNSUPPORTED,
               "fg_plan_single_optim: Adam keeps one step counter per plan; use fg_plan_optim");
    return run_optim(*p, p->mt_single[input_index]);
}

FG_API int fg_plan_capture_step(fg_plan *p) {
    FG_REQUIRE(p && p->ctx, FG_ERR_INVALID_ARGUMENT, "fg_plan_capture_step: plan is NULL or has no device (dry plan)");
    FG_HIP(hipSetDevice(p->ctx->device));
    for (size_t k = 0; k < p->inputs.size(); ++k)
        FG_REQUIRE(p->ptr(p->input_slot[k]), FG_ERR_INVALID_ARGUMENT,
                   "fg_plan_capture_step: input %zu is not bound", k);
    FG_REQUIRE(p->ptr(p->target_slot), FG_ERR_INVALID_ARGUMENT,
               "fg_plan_capture_step: no target bound");
    int rc = ensure_mt(*p);  // allocates: must precede capture
    if (rc) return rc;
    rc = prepare_elt(*p, {&p->fwd, &p->loss, &p->bwd_fused, &p->bwd_seed});
    if (rc) return rc;
    drop_graph(*p);
    FG_HIP(hipStreamSynchronize(p->ctx->stream));
    FG_HIP(hipStreamBeginCapture(p->ctx->stream, hipStreamCaptureModeThreadLocal));
    // With SGD the head GEMM may finish the loss (its mean then runs in the
    // SGD launch).
    const int hc = head_loss_chain(*p);
    const bool overlap = p->g.optim == FG_OPTIM_ADAM && !p->mt_groups.empty();
    p->hold_mean = overlap;
    const std::vector<Launch> &bwd = p->ce_fused_possible ? p->bwd_fused : p->bwd_seed;
    const bool hb = head_bwd_fusable(*p, bwd, hc);
    bool ce_done = false;
    rc = run(*p, p->fwd, true, false, hc >= 0 ? &p->loss[0] : nullptr, &ce_done,
             hb ? &bwd[1] : nullptr);
    if (rc == FG_OK && ce_done) {
        const Launch &S = p->loss[0];
        p->wctx.mean_src = (const float *)p->ptr(S.sB);
        p->wctx.mean_dst = (float *)p->ptr(S.sBias);
        p->wctx.mean_rows = S.M;
    } else if (rc == FG_OK) {
        rc = run(*p, p->loss, true);
    }
    // The backward's last summing launch may share the SGD launch; with the
    // head's dX computed in the forward, the head's dW runs beside the next
    // pair.
    if (rc == FG_OK && overlap) {
        rc = run_bwd_adam_overlapped(*p, bwd);
    } else {
        if (rc == FG_OK)
            rc = run(*p, bwd, false, p->g.optim == FG_OPTIM_SGD && p->mt_all, nullptr, nullptr,
                     nullptr, ce_done && hb ? 0 : -1);
        if (rc == FG_OK) rc = run_optim(*p, p->mt_all);
    }
    p->wctx.defer_reduce = false;
    p->hold_mean = false;
    if (rc != FG_OK) {
        p->wctx.pending_splits = 0;
        p->wctx.mean_dst = nullptr;
    }
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(p->ctx->stream, &graph);
    if (rc != FG_OK) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc;
    }
    if (e != hipSuccess) return fg::hip_fail(e, "hipStreamEndCapture", __FILE__, __LINE__);
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return fg::hip_fail(e, "hipGraphInstantiate", __FILE__, __LINE__);
    }
    p->graph = graph;
    p->exec = exec;
    return FG_OK;
}

FG_API int fg_plan_launch_step(fg_plan *p) {
    FG_REQUIRE(p && p->ctx, FG_ERR_INVALID_ARGUMENT, "fg_plan_launch_step: plan is NULL or has no device (dry plan)");
    FG_REQUIRE(p->exec, FG_ERR_INVALID_ARGUMENT,
               "fg_plan_launch_step: no captured step (call fg_plan_capture_step; rebinding "
               "inputs, target or hyper-parameters drops the capture)");
    FG_HIP(hipSetDevice(p->ctx->device));
    FG_HIP(hipGraphLaunch(p->exec, p->ctx->stream));
    return FG_OK;
}

// ------------------------------------------------------------ checkpoints
// A checkpoint is a bpat file holding every Input in input order, then for
// Adam the m and v state of each updated input and a one-element tensor
// with the step count (the reference's io::save_tensors covers the tensors
// a caller passes; optimiser state has no counterpart there).
namespace {
int plan_ckpt_tensors(const fg_plan *p, std::vector<fg_bpat_tensor> &ts) {
    auto add = [&](int slot, uint32_t node) -> int {
        fg_bpat_tensor t{};
        t.d_ptr = p->ptr(slot);
        FG_REQUIRE(t.d_ptr, FG_ERR_INVALID_ARGUMENT,
                   "checkpoint: input node %u is not bound", node);
        t.dtype = p->slots[slot].dtype;
        const Shape &sh = p->shape[node];
        if (sh.vector) {
            t.rank = 1;
            t.shape[0] = (uint32_t)sh.cols;
        } else {
            t.rank = 2;
            t.shape[0] = (uint32_t)sh.rows;
            t.shape[1] = (uint32_t)sh.cols;
        }
        ts.push_back(t);
        return FG_OK;
    };
    for (size_t k = 0; k < p->inputs.size(); ++k)
        if (int rc = add(p->input_slot[k], p->inputs[k])) return rc;
    if (p->g.optim == FG_OPTIM_ADAM) {
        for (uint32_t k : p->opt_inputs) {
            if (int rc = add(p->m_slot[k], p->inputs[k])) return rc;
            ts.back().dtype = FG_DTYPE_F32;
            if (int rc = add(p->v_slot[k], p->inputs[k])) return rc;
            ts.back().dtype = FG_DTYPE_F32;
        }
    }
    return FG_OK;
}
}  // namespace

FG_API int fg_plan_save(fg_plan *p, const char *path, int header) {
    FG_REQUIRE(p && p->ctx && path, FG_ERR_INVALID_ARGUMENT, "fg_plan_save: NULL argument");
    std::vector<fg_bpat_tensor> ts;
    if (int rc = plan_ckpt_tensors(p, ts)) return rc;
    float step = 0.0f;
    if (p->g.optim == FG_OPTIM_ADAM) {
        uint32_t st[4];
        FG_HIP(hipSetDevice(p->ctx->device));
        FG_HIP(hipMemcpyAsync(st, p->ptr(p->adam_slot), sizeof st, hipMemcpyDeviceToHost,
                              p->ctx->stream));
        FG_HIP(hipStreamSynchronize(p->ctx->stream));
        step = (float)st[0];
    }
    // Host copies of every tensor, then one write (with the step count last).
    std::vector<fg_bpat_tensor> all;
    std::vector<std::vector<uint8_t>> host(ts.size());
    FG_HIP(hipSetDevice(p->ctx->device));
    for (size_t i = 0; i < ts.size(); ++i) {
        uint64_t n = 1;
        for (int d = 0; d < ts[i].rank; ++d) n *= ts[i].shape[d];
        host[i].resize(n * esize(ts[i].dtype));
        if (n)
            FG_HIP(hipMemcpyAsync(host[i].data(), ts[i].d_ptr, host[i].size(),
                                  hipMemcpyDeviceToHost, p->ctx->stream));
        fg_bpat_tensor h = ts[i];
        h.d_ptr = host[i].data();
        all.push_back(h);
    }
    FG_HIP(hipStreamSynchronize(p->ctx->stream));
    if (p->g.optim == FG_OPTIM_ADAM) {
        fg_bpat_tensor s{};
        s.d_ptr = &step;
        s.dtype = FG_DTYPE_F32;
        s.rank = 1;
        s.shape[0] = 1;
        all.push_back(s);
    }
    return fg_bpat_save_host(path, header, (int)all.size(), all.data());
}

FG_API int fg_plan_load(fg_plan *p, const char *path) {
    FG_REQUIRE(p && p->ctx && path, FG_ERR_INVALID_ARGUMENT, "fg_plan_load: NULL argument");
    std::vector<fg_bpat_tensor> ts;
    if (int rc = plan_ckpt_tensors(p, ts)) return rc;
    fg_bpat *f = nullptr;
    if (int rc = fg_bpat_open(path, &f)) return rc;
    std::unique_ptr<fg_bpat, int (*)(fg_bpat *)> guard(f, fg_bpat_close);
    int count = 0;
    fg_bpat_info(f, nullptr, &count);
    const bool adam = p->g.optim == FG_OPTIM_ADAM;
    FG_REQUIRE(count == (int)ts.size() + (adam ? 1 : 0), FG_ERR_SHAPE,
               "fg_plan_load: %s holds %d tensors, the plan expects %zu", path, count,
               ts.size() + (adam ? 1 : 0));
    for (size_t i = 0; i < ts.size(); ++i) {
        uint64_t n = 0, want = 1;
        fg_bpat_tensor_info(f, (int)i, nullptr, nullptr, &n);
        for (int d = 0; d < ts[i].rank; ++d) want *= ts[i].shape[d];
        FG_REQUIRE(n == want, FG_ERR_SHAPE, "fg_plan_load: tensor %zu has %llu elements, not %llu",
                   i, (unsigned long long)n, (unsigned long long)want);
    }
    for (size_t i = 0; i < ts.size(); ++i)
        if (int rc = fg_bpat_upload(p->ctx, f, (int)i, const_cast<void *>(ts[i].d_ptr),
                                    ts[i].dtype))
            return rc;
    if (adam) {
        uint64_t n = 0;
        fg_bpat_tensor_info(f, (int)ts.size(), nullptr, nullptr, &n);
        FG_REQUIRE(n == 1, FG_ERR_SHAPE, "fg_plan_load: the step-count tensor has %llu elements",
                   (unsigned long long)n);
        float step = 0.0f;
        fg_bpat_read_f32(f, (int)ts.size(), &step);
        FG_REQUIRE(step >= 0.0f && step < 4294967296.0f && step == std::floor(step),
                   FG_ERR_SERIALIZATION, "fg_plan_load: step count %g is not a count", step);
        const uint32_t st[4] = {(uint32_t)step, 0u, 0u, 0u};
        FG_HIP(hipSetDevice(p->ctx->device));
        FG_HIP(hipMemcpyAsync(p->ptr(p->adam_slot), st, sizeof st, hipMemcpyHostToDevice,
                              p->ctx->stream));
        FG_HIP(hipStreamSynchronize(p->ctx->stream));
    }
    return FG_OK;
}

FG_API int fg_plan_describe(const fg_plan *p, char *buf, size_t len, size_t *needed) {
    FG_REQUIRE(p, FG_ERR_INVALID_ARGUMENT, "fg_plan_describe: plan is NULL");
    std::string s;
    fg_ctx *wc = p->ctx ? const_cast<fg_ctx *>(&p->wctx) : nullptr;
    // Dispatches of a GEMM launch: 2 when K is split (the slices, then the
    // kernel that sums them in slice order and applies the epilogue).
    auto gemm_dispatches = [&](const Launch &L) {
        if (L.kind != LK_GEMM && L.kind != LK_GEMM_BWD) return 1;
        if (L.dtype != FG_DTYPE_F32)
            return fg::gemm16_dispatches(wc, L.sExtra != kNone ? FG_TN : L.layout, L.M, L.N, L.K,
                                         p->ptr(L.sA), L.lda, p->ptr(L.sB), L.ldb,
                                         L.kind == LK_GEMM && L.sExtra != kNone);
        return fg::gemm_f32_dispatches(wc, L.sExtra != kNone ? FG_TN : L.layout, L.M, L.N, L.K,
                                       p->ptr(L.sA), L.lda, p->ptr(L.sB), L.ldb,
                                       L.kind == LK_GEMM && L.sExtra != kNone);
    };
    // Dispatches of a forward chain (L and the next launch X).
    auto chain_dispatches = [&](const Launch &L, const Launch &X) {
        if (!wc) return gemm_dispatches(L) + gemm_dispatches(X);
        return fg::gemm_fwd_chain_dispatches(
            wc, L.M, L.N, L.K, p->ptr(L.sA), L.lda, p->ptr(L.sB), L.ldb, p->ptr(L.sBias),
            p->ptr(L.sC), L.ldc, p->ptr(L.sZ), L.ldz, X.M, X.N, X.K, p->ptr(X.sA), X.lda,
            p->ptr(X.sB), X.ldb);
    };
    auto add = [&](const char *title, const std::vector<Launch> &v) {
        s += std::string(title) + ": " + std::to_string(v.size()) + " launches\n";
        for (size_t i = 0; i < v.size(); ++i) {
            const Launch &L = v[i];
            s += "  " + L.desc;
            const int nd = gemm_dispatches(L);
            if (nd == 3) {  // a 16-bit dW off the pipelined kernel
                s += " [GEMM + column-sum reduction]";
            } else if (nd > 1) {
                const bool summed_by_next = L.chain_next && i + 1 < v.size() &&
                                            chain_dispatches(L, v[i + 1]) == 2;
                s += summed_by_next ? " [K split: slices, summed by the next launch]"
                                    : " [K split: slices + summing kernel]";
            }
            s += "\n";
        }
    };
    // Kernel dispatches per planned launch in a captured step: the
    // bias-gradient reduction is a partial and a final pass, a GEMM that
    // splits K adds its summing kernel, the fused softmax + CE adds the
    // mean-loss reduction unless its one-workgroup form computes the mean,
    // the final forward softmax is left to the loss launch, the Adam update
    // is preceded by its step-counter advance.
    auto kernels = [&](const std::vector<Launch> &v) {
        int n = 0;
        for (size_t i = 0; i < v.size(); ++i) {
            const Launch &L = v[i];
            if (L.elidable) continue;
            if (L.chain_next && i + 1 < v.size()) {
                n += chain_dispatches(L, v[i + 1]);
                ++i;
            } else if (L.pair_next && i + 1 < v.size() && L.dtype != FG_DTYPE_F32) {
                const Launch &X = v[i + 1];
                n += wc ? fg::gemm16_dw_dx_dispatches(wc, L.M, L.N, L.K, p->ptr(L.sA), L.lda,
                                                      p->ptr(L.sB), L.ldb, X.M, X.N, X.K,
                                                      p->ptr(X.sA), X.lda, p->ptr(X.sB), X.ldb)
                        : gemm_dispatches(L) + gemm_dispatches(X);
                ++i;
            } else if (L.pair_next && i + 1 < v.size()) {
                const Launch &X = v[i + 1];
                n += wc ? fg::gemm_dw_dx_dispatches(wc, L.M, L.N, L.K, p->ptr(L.sA), L.lda,
                                                    p->ptr(L.sB), L.ldb, X.M, X.N, X.K,
                                                    p->ptr(X.sA), X.lda, p->ptr(X.sB), X.ldb)
                        : gemm_dispatches(L) + gemm_dispatches(X);
                ++i;
            } else if (L.kind == LK_SMCE)
                n += fg::softmax_ce_dispatches(L.M, L.N, L.sBias != kNone);
            else if (L.kind == LK_BIAS_GRAD)
                n += 2;
            else
                n += gemm_dispatches(L);
        }
        return n;
    };
    add("forward", p->fwd);
    add("loss", p->loss);
    add("backward(seed)", p->bwd_seed);
    if (p->ce_fused_possible) add("backward(ce-fused)", p->bwd_fused);
    const bool adam = p->g.optim == FG_OPTIM_ADAM;
    s += "optim: " + std::string(adam ? "adam" : "sgd") + " over " +
         std::to_string(p->opt_inputs.size()) + " inputs, 1 multi-tensor launch\n";
    int k_opt = p->opt_inputs.empty() ? 0 : (adam ? 2 : 1);
    bool opt_f32 = true;
    for (uint32_t idx : p->opt_inputs) opt_f32 = opt_f32 && p->dtype[p->inputs[idx]] == FG_DTYPE_F32;
    if (adam && wc && opt_f32 && !p->opt_inputs.empty()) {
        // Captured: the step counter, then one update per group of inputs
        // the backward releases together (run_bwd_adam_overlapped).
        const std::vector<int> after = adam_group_after(*p);
        const int groups = (int)std::set<int>(after.begin(), after.end()).size();
        k_opt = 1 + groups;
        s += "(captured step: the Adam update runs in " + std::to_string(groups) +
             " launches on a second stream, each once the backward is done with its "
             "tensors)\n";
    }
    const std::vector<Launch> &bwd = p->ce_fused_possible ? p->bwd_fused : p->bwd_seed;
    int k_bwd = kernels(bwd);
    int k_loss = kernels(p->loss);
    // A captured SGD step may finish the loss in the head GEMM, and then the
    // head's data gradient too, its dW joining the next pair's launch.
    if (const int hc = head_loss_chain(*p); hc >= 0 && wc &&
                                            chain_dispatches(p->fwd[hc], p->fwd[hc + 1]) == 2) {
        k_loss = 0;
        s += "(captured step: the head GEMM finishes the loss; its mean runs in the SGD launch)\n";
        if (head_bwd_fusable(*p, bwd, hc)) {
            auto pair_n = [&](const Launch &L, const Launch &X) {
                return fg::gemm_dw_dx_dispatches(wc, L.M, L.N, L.K, p->ptr(L.sA), L.lda,
                                                 p->ptr(L.sB), L.ldb, X.M, X.N, X.K,
                                                 p->ptr(X.sA), X.lda, p->ptr(X.sB), X.ldb);
            };
            const Launch &W0 = bwd[0], &W1 = bwd[2], &D1 = bwd[3];
            const int triple = fg::gemm_dw_dw_dx_dispatches(
                wc, W0.M, W0.N, W0.K, p->ptr(W0.sA), W0.lda, p->ptr(W0.sB), W0.ldb, W1.M, W1.N,
                W1.K, p->ptr(W1.sA), W1.lda, p->ptr(W1.sB), W1.ldb, D1.M, D1.N, D1.K,
                p->ptr(D1.sA), D1.lda, p->ptr(D1.sB), D1.ldb);
            k_bwd += triple - pair_n(bwd[0], bwd[1]) - pair_n(bwd[2], bwd[3]);
            s += "(captured step: it also computes the head's data gradient; the head's dW "
                 "runs in the next pair's launch)\n";
        }
    }
    // A captured SGD step runs the backward's last summing launch beside the
    // SGD update (run_optim), when the two touch disjoint memory.
    if (!adam && wc && !p->opt_inputs.empty() && !bwd.empty()) {
        const Launch &X = bwd.back();
        const Launch *L = bwd.size() >= 2 && bwd[bwd.size() - 2].pair_next ? &bwd[bwd.size() - 2]
                                                                           : nullptr;
        // (fp32 summing passes only: a 16-bit split sums within its own call)
        auto held = [&](const Launch *G) {
            return G && G->dtype == FG_DTYPE_F32 && gemm_dispatches(*G) > 1;
        };
        const Launch *H = held(&X) ? &X : held(L) ? L : nullptr;
        if (H) {
            auto slot_range = [&](int slot) {
                const uintptr_t b0 = (uintptr_t)p->ptr(slot);
                return fg::ByteRange{b0, b0 + p->slots[slot].bytes};
            };
            std::vector<fg::ByteRange> held = {slot_range(H->sC)};
            if (H->kind == LK_GEMM_BWD && H->act != FG_ACT_NONE) held.push_back(slot_range(H->sZ));
            bool shared = true;
            for (const fg::ByteRange &o : optim_ranges(*p))
                for (const fg::ByteRange &q : held) shared = shared && !q.overlaps(o);
            if (shared) {
                --k_bwd;
                s += "(captured step: the backward's last summing launch shares the SGD launch)\n";
            }
        }
    }
    s += "kernels per step: " +
         std::to_string(kernels(p->fwd) + k_loss + k_bwd + k_opt) +
         " (forward " + std::to_string(kernels(p->fwd)) + ", loss " +
         std::to_string(k_loss) + ", backward " + std::to_string(k_bwd) +
         ", optim " + std::to_string(k_opt) + ")\n";
    s += "arena: " + std::to_string(p->arena_bytes) + " bytes\n";
    if (needed) *needed = s.size() + 1;
    if (buf && len) {
        const size_t n = std::min(len - 1, s.size());
        std::memcpy(buf, s.data(), n);
        buf[n] = 0;
    }
    return FG_OK;
}
