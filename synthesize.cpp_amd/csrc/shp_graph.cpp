// Node-run executor: splits an ordered ggml-style node list into runs (a fused
// run where the reference's graphs emit one, else one node at a time) and
// launches each through the entry points of synth_hip.h.
//
// A run is recognised from its last node (its result) backwards through the
// src_node links, and is taken only when the nodes it reaches are exactly the
// next nodes of the list (view-like nodes aside) and every intermediate result
// it does not write is read by nothing outside the run and is not a graph
// output. That is the condition under which skipping the intermediate writes
// cannot be observed. Every fused launch computes what the nodes compute one
// by one, bit for bit.
#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <initializer_list>
#include <vector>

#include "shp_internal.hpp"
#include "synth_graph.h"
#include "synth_hip.h"

namespace shp {
namespace {

float fparam(const shp_node & n, int i) {
    float f;
    std::memcpy(&f, &n.op_params[i], sizeof(f));
    return f;
}

bool present(const shp_tensor & t) {
    return t.data != nullptr;
}

// The same tensor: same memory, shape and strides.
bool same_tensor(const shp_tensor & a, const shp_tensor & b) {
    return a.data == b.data && a.type == b.type && same_shape(a, b) && a.nb[0] == b.nb[0] && a.nb[1] == b.nb[1] &&
           a.nb[2] == b.nb[2] && a.nb[3] == b.nb[3];
}

bool f32_of(const shp_tensor & t) {
    return well_formed(&t) && t.type == SHP_TYPE_F32 && t.ne[0] <= INT32_MAX;
}

// ggml_mul / ggml_add / ggml_div operand b as the fused runs take it: a's
// shape, or one row of a.ne[0] elements repeated over a's rows.
bool row_operand(const shp_tensor & a, const shp_tensor & b) {
    return f32_of(b) && (same_shape(a, b) || one_row_of(b, a.ne[0]));
}

// A gain vector of n elements, as ggml_mul repeats it: F32, BF16 or F16,
// [n, 1, 1, 1]. (Another shape of n elements, [1, n] say, ggml repeats
// differently.)
bool gain_vector(const shp_tensor & w, int64_t n) {
    return well_formed(&w) && weight_kind(w.type) >= 0 && one_row_of(w, n);
}

bool unary_ok(const shp_node & n) {
    return f32_of(n.src[0]) && f32_of(n.dst) && same_shape(n.src[0], n.dst);
}

// A single binary node also takes every other b that repeats to a's shape.
bool binary_ok(const shp_node & n) {
    return f32_of(n.src[0]) && f32_of(n.dst) && same_shape(n.src[0], n.dst) &&
           (row_operand(n.src[0], n.src[1]) || (f32_of(n.src[1]) && can_repeat(n.src[1], n.src[0])));
}

bool rope_params_ok(const shp_node & n) {
    const int32_t n_dims = n.op_params[1];
    const int32_t mode   = n.op_params[2];
    const auto &  x      = n.src[0];
    const auto &  pos    = n.src[1];
    return mode == SHP_ROPE_TYPE_NEOX && fparam(n, 7) == 0.0f && !present(n.src[2]) && f32_of(x) && f32_of(n.dst) &&
           same_shape(x, n.dst) && x.ne[3] == 1 && well_formed(&pos) && pos.type == SHP_TYPE_I32 &&
           nelements(pos) == x.ne[2] && contiguous(pos) && n_dims > 0 && n_dims % 2 == 0 && n_dims <= x.ne[0];
}

shp_status_t launch_single(const shp_node & n, shp_stream_t st);

// The ggml node's own fields an entry point does not see: sources present
// and well formed, op parameters this library implements (no ALiBi, no rope
// frequency factors, no softmax sinks).
bool node_form_ok(const shp_node & n) {
    // A copy may read a transposed or permuted F32 view (rows not contiguous).
    const bool strided_src = n.op == SHP_NODE_CPY && f32_strided_view_dim(&n.src[0]) != 0;
    for (int k = strided_src ? 1 : 0; k < SHP_NODE_MAX_SRC; ++k) {
        if (present(n.src[k]) && !well_formed(&n.src[k])) {
            return false;
        }
    }
    switch (n.op) {
        case SHP_NODE_NOP:
            return true;
        case SHP_NODE_ADD:
        case SHP_NODE_MUL:
        case SHP_NODE_DIV:
        case SHP_NODE_SUB:
            return binary_ok(n);
        case SHP_NODE_SQR:
        case SHP_NODE_SIN:
        case SHP_NODE_SILU:
        case SHP_NODE_EXP:
        case SHP_NODE_LEAKY_RELU:
        case SHP_NODE_SCALE:
        case SHP_NODE_TANH:
        case SHP_NODE_SIGMOID:
        case SHP_NODE_ELU:
        case SHP_NODE_GELU_ERF:
        case SHP_NODE_CLAMP:
        case SHP_NODE_RELU:
        case SHP_NODE_NEG:
        case SHP_NODE_STEP:
        case SHP_NODE_SQRT:
            return unary_ok(n);
        case SHP_NODE_DIAG_MASK_INF:
            return unary_ok(n) && n.op_params[0] >= 0;
        case SHP_NODE_SUM_ROWS:
        case SHP_NODE_MEAN:
            return f32_of(n.src[0]) && f32_of(n.dst) && n.dst.ne[0] == 1 && n.dst.ne[1] == n.src[0].ne[1] &&
                   n.dst.ne[2] == n.src[0].ne[2] && n.dst.ne[3] == n.src[0].ne[3];
        case SHP_NODE_NORM:
            return unary_ok(n) && fparam(n, 0) >= 0.0f;
        case SHP_NODE_CPY:
            return (strided_src || (well_formed(&n.src[0]) && (n.src[0].type == SHP_TYPE_F32 ||
                                                                n.src[0].type == SHP_TYPE_F16 ||
                                                                n.src[0].type == SHP_TYPE_BF16))) &&
                   f32_of(n.dst) && same_shape(n.src[0], n.dst);
        case SHP_NODE_GET_ROWS: {
            const auto & t   = n.src[0];
            const auto & ids = n.src[1];
            const bool   tt  = t.type == SHP_TYPE_F32 || t.type == SHP_TYPE_F16 || t.type == SHP_TYPE_BF16 ||
                            t.type == SHP_TYPE_Q8_0 || t.type == SHP_TYPE_Q5_K;
            return well_formed(&t) && tt && well_formed(&ids) && ids.type == SHP_TYPE_I32 && f32_of(n.dst) &&
                   n.dst.ne[0] == t.ne[0] && n.dst.ne[1] == ids.ne[0] && n.dst.ne[2] == ids.ne[1] &&
                   n.dst.ne[3] == ids.ne[2] && ids.ne[3] == 1;
        }
        case SHP_NODE_RMS_NORM:
            return unary_ok(n) && fparam(n, 0) >= 0.0f;
        case SHP_NODE_SOFT_MAX: {
            const auto & m = n.src[1];
            return unary_ok(n) && fparam(n, 1) == 0.0f && !present(n.src[2]) &&
                   (!present(m) || (f32_of(m) && m.ne[0] == n.src[0].ne[0] && m.ne[1] >= n.src[0].ne[1]));
        }
        case SHP_NODE_ROPE:
            return rope_params_ok(n);
        case SHP_NODE_CONCAT:
            return f32_of(n.src[0]) && f32_of(n.src[1]) && f32_of(n.dst) && n.op_params[0] >= 0 &&
                   n.op_params[0] <= 3;
        case SHP_NODE_COL2IM_1D:
            return f32_of(n.src[0]) && f32_of(n.dst);
        case SHP_NODE_PAD: {
            // {lp0, rp0, ..., lp3, rp3}; no circular padding; the extents add up
            if (n.op_params[8] != 0 || !f32_of(n.src[0]) || !f32_of(n.dst)) {
                return false;
            }
            for (int d = 0; d < 4; ++d) {
                const int32_t lp = n.op_params[2 * d], rp = n.op_params[2 * d + 1];
                if (lp < 0 || rp < 0 || n.dst.ne[d] != n.src[0].ne[d] + lp + rp) {
                    return false;
                }
            }
            return true;
        }
        case SHP_NODE_PAD_REFLECT_1D:
        case SHP_NODE_REPEAT:
            return f32_of(n.src[0]) && f32_of(n.dst);
        case SHP_NODE_ACC:
            // {nb1, nb2, nb3, offset, inplace}: ggml's view of the result
            return f32_of(n.src[0]) && f32_of(n.src[1]) && f32_of(n.dst) && same_shape(n.src[0], n.dst) &&
                   n.op_params[0] >= 0 && n.op_params[1] >= 0 && n.op_params[2] >= 0 && n.op_params[3] >= 0;
        case SHP_NODE_IM2COL:
            // the 1-D form: is_2D 0 and no padding along the absent second
            // dimension (ggml's 1-D rows read there at -p1: zeros)
            return n.op_params[6] == 0 && n.op_params[3] == 0 && present(n.src[0]) && f32_of(n.src[1]) &&
                   (n.dst.type == SHP_TYPE_F32 || n.dst.type == SHP_TYPE_F16);
        case SHP_NODE_GLU_SWIGLU: {
            const auto & a = n.src[0];
            if (!f32_of(a) || !f32_of(n.dst)) {
                return false;
            }
            if (present(n.src[1])) {
                return same_shape(a, n.src[1]) && f32_of(n.src[1]) && same_shape(a, n.dst);
            }
            return a.ne[0] % 2 == 0 && n.dst.ne[0] * 2 == a.ne[0] && n.dst.ne[1] == a.ne[1] &&
                   n.dst.ne[2] == a.ne[2] && n.dst.ne[3] == a.ne[3];
        }
        default:
            return false;
    }
}

// A node runs alone when its form is one this library implements and its
// entry point, called in a dry run, accepts its operands: supports_op == 1
// then means the launch goes through.
bool single_ok(const shp_node & n) {
    if (!node_form_ok(n)) {
        return false;
    }
    DryRun dry;
    return launch_single(n, nullptr) == SHP_OK;
}

// The nodes of a candidate run (at most 2*64 - 1: the longest gather->sum).
struct Members {
    int v[128];
    int n = 0;
    Members() = default;
    Members(std::initializer_list<int> xs) {
        for (int x : xs) {
            v[n++] = x;
        }
    }
    void push(int x) { v[n++] = x; }
    int  back() const { return v[n - 1]; }
    bool has(int x) const {
        for (int i = 0; i < n; ++i) {
            if (v[i] == x) {
                return true;
            }
        }
        return false;
    }
};

// What a run launches: which entry point, and its operands. The q/k runs put
// k's operands in x2/w2/y2 and v's copy in x3/y3.
struct Launch {
    int                     kind  = SHP_RUN_SINGLE;
    int                     first = 0;
    int                     last  = 0;
    int                     count = 0;
    const shp_tensor *      x     = nullptr;
    const shp_tensor *      b     = nullptr;
    const shp_tensor *      w     = nullptr;
    const shp_tensor *      c1    = nullptr;
    shp_tensor *            y     = nullptr;
    shp_tensor *            sum   = nullptr;
    const shp_tensor *      x2    = nullptr;
    const shp_tensor *      w2    = nullptr;
    shp_tensor *            y2    = nullptr;
    const shp_tensor *      x3    = nullptr;
    shp_tensor *            y3    = nullptr;
    float                   f0    = 0.0f;
    float                   f1    = 0.0f;
    float                   f2    = 0.0f;
    int32_t                 i0    = 0;
    int32_t                 i1    = 0;
    int32_t                 i2    = 0;
    std::vector<shp_tensor> terms;
    shp_tensor              codes{};
    // views the run forms itself (a transposed view of a copy's source, a
    // [1, C] bias read as one row of C): used in place of x / b when set
    shp_tensor              xv{};
    shp_tensor              bv{};
    bool                    own_x = false;
    bool                    own_b = false;
};

class Planner;
shp_status_t launch_run(const Planner & pl, const Launch & l, shp_stream_t st);

class Planner {
  public:
    Planner(const shp_node * nodes, int n) : nodes_(nodes), n_(n) {}

    // Checks the list and indexes each node's readers (one entry per src
    // reference, in a flat array: cons_[cstart_[j] .. cstart_[j + 1])).
    shp_status_t init() {
        cstart_.assign(n_ + 1, 0);
        for (int i = 0; i < n_; ++i) {
            const shp_node & nd = nodes_[i];
            if (nd.uses < 0 || nd.op < 0 || nd.op >= SHP_NODE_OP_COUNT) {
                return SHP_ERR_INVALID_ARG;
            }
            for (int k = 0; k < SHP_NODE_MAX_SRC; ++k) {
                const int j = nd.src_node[k];
                if (j == -1) {
                    continue;
                }
                if (j < 0 || j >= i || !present(nd.src[k])) {
                    return SHP_ERR_INVALID_ARG;
                }
                ++cstart_[j + 1];
            }
            if (nd.op != SHP_NODE_NOP) {
                order_.push_back(i);
            }
        }
        for (int j = 0; j < n_; ++j) {
            cstart_[j + 1] += cstart_[j];
        }
        cons_.assign(cstart_[n_], 0);
        std::vector<int> fill(cstart_.begin(), cstart_.end() - 1);
        for (int i = 0; i < n_; ++i) {
            for (int k = 0; k < SHP_NODE_MAX_SRC; ++k) {
                const int j = nodes_[i].src_node[k];
                if (j >= 0) {
                    cons_[fill[j]++] = i;
                }
            }
        }
        for (int j = 0; j < n_; ++j) {
            if (nodes_[j].uses != 0 && nodes_[j].uses < readers(j)) {
                return SHP_ERR_INVALID_ARG;
            }
        }
        return SHP_OK;
    }

    // Every run of the list, in launch order; NOP nodes are runs of their own,
    // placed by index. The parts of a q/k run that sat later in the list leave
    // the window order once taken, so later windows see the list without them.
    std::vector<Launch> plan() {
        std::vector<Launch> out;
        int                 nop = 0;
        auto                nops_before = [&](int upto) {
            for (; nop < upto; ++nop) {
                if (nodes_[nop].op == SHP_NODE_NOP) {
                    Launch v;
                    v.kind  = SHP_RUN_NOP;
                    v.first = v.last = nop;
                    out.push_back(v);
                }
            }
        };
        size_t p = 0;
        while (p < order_.size()) {
            const int i = order_[p];
            nops_before(i);
            Launch l;
            int    used = match(p, l);
            if (used > 0) {
                // a fused run is taken only when its entry point accepts the
                // operands and its outputs are apart from what it reads;
                // otherwise its nodes run one by one
                DryRun dry;
                if (launch_run(*this, l, nullptr) != SHP_OK || !io_apart(p, used, l)) {
                    used = 0;
                }
            }
            if (used == 0) {
                l       = Launch{};
                l.kind  = single_ok(nodes_[i]) ? SHP_RUN_SINGLE : SHP_RUN_UNSUPPORTED;
                l.first = l.last = i;
                l.count          = 1;
                out.push_back(l);
                ++p;
                continue;
            }
            l.first = order_[p];
            l.last  = order_[p + used - 1];
            l.count = used;
            if (l.kind == SHP_RUN_NORM_MUL_ROPE) {
                Launch qk;
                if (match_sibling(p, used, l, qk)) {
                    l = qk;
                }
            }
            out.push_back(l);
            p += used;
        }
        nops_before(n_);
        return out;
    }

    const shp_node & node(int i) const { return nodes_[i]; }

  private:
    // A run writes its outputs in one launch while it reads its inputs. The
    // allocator may give an output the memory of a tensor that a node of the
    // run read last (freed once that node had run), so an output may overlap
    // an input at another offset or stride: the launch would then read values
    // it has already overwritten. The run is taken only when every output is
    // apart from every tensor the run reads from outside, or is that very
    // tensor (the same bytes and strides: each kernel reads an element or a
    // row before it writes it).
    bool io_apart(size_t p, int used, const Launch & l) const {
        Members members;
        for (int k = 0; k < used; ++k) {
            members.push(order_[p + k]);
        }
        const shp_tensor * outs[] = { l.y, l.y2, l.y3, l.sum };
        for (int a = 0; a < members.n; ++a) {
            const int m = members.v[a];
            for (int k = 0; k < SHP_NODE_MAX_SRC; ++k) {
                const shp_tensor & in = nodes_[m].src[k];
                if (!present(in) || members.has(producer(m, k))) {
                    continue;
                }
                for (const shp_tensor * o : outs) {
                    if (o != nullptr && spans_overlap(in, *o) && !same_tensor(in, *o)) {
                        return false;
                    }
                }
            }
        }
        return true;
    }

    // Window positions scanned past a rope run for its sibling and v's copy.
    static constexpr size_t kSiblingScan = 64;

    // A byte range [lo, hi) of device memory.
    struct Span {
        uintptr_t lo;
        uintptr_t hi;
    };

    // The bytes a descriptor can address: from data to the end of its last
    // element (of its last row, for a block type). A strided view's ne[0]
    // counts through nb[0].
    static Span extent(const shp_tensor & t) {
        Span sp;
        byte_span(t, sp.lo, sp.hi);
        return sp;
    }

    static bool overlaps(const Span & a, const std::vector<Span> & bs) {
        for (const Span & b : bs) {
            if (a.lo < b.hi && b.lo < a.hi) {
                return true;
            }
        }
        return false;
    }

    // The producer of src k of node m, seen through view-like nodes (-1: none
    // in the list).
    int producer(int m, int k) const {
        int j = nodes_[m].src_node[k];
        while (j >= 0 && nodes_[j].op == SHP_NODE_NOP) {
            j = nodes_[j].src_node[0];
        }
        return j;
    }

    // One part of a q/k run: its nodes, the ranges it reads from outside
    // itself and the one range it writes (its sink's dst).
    struct Part {
        Members           nodes;
        std::vector<Span> reads;
        std::vector<Span> writes;
        size_t            pos = 0;  // window position of its first node
    };

    Part part_of(size_t p, int used, int sink) const {
        Part pt;
        pt.pos = p;
        for (int k = 0; k < used; ++k) {
            pt.nodes.push(order_[p + k]);
        }
        for (int a = 0; a < pt.nodes.n; ++a) {
            const int m = pt.nodes.v[a];
            for (int k = 0; k < SHP_NODE_MAX_SRC; ++k) {
                if (present(nodes_[m].src[k]) && !pt.nodes.has(producer(m, k))) {
                    pt.reads.push_back(extent(nodes_[m].src[k]));
                }
            }
        }
        pt.writes.push_back(extent(nodes_[sink].dst));
        return pt;
    }

    // A part that sits later in the list can run at window position `at`
    // instead: every input it takes from the list is produced before `at`
    // (or is its own), and no node between `at` and the part (other than the
    // members of the whole run) writes what it reads or writes, or reads what
    // it writes -- so moving it up changes no value any node sees.
    bool can_move_up(const Part & pt, size_t at, const Members & all) const {
        const int first = order_[at];
        for (int a = 0; a < pt.nodes.n; ++a) {
            const int m = pt.nodes.v[a];
            for (int k = 0; k < SHP_NODE_MAX_SRC; ++k) {
                const int j = producer(m, k);
                if (j >= first && !pt.nodes.has(j)) {
                    return false;
                }
            }
        }
        for (size_t q = at + 1; q < pt.pos; ++q) {
            const int x = order_[q];
            if (all.has(x)) {
                continue;
            }
            const shp_node & X = nodes_[x];
            const Span       w = extent(X.dst);
            if (overlaps(w, pt.reads) || overlaps(w, pt.writes)) {
                return false;
            }
            for (int k = 0; k < SHP_NODE_MAX_SRC; ++k) {
                if (present(X.src[k]) && overlaps(extent(X.src[k]), pt.writes)) {
                    return false;
                }
            }
        }
        return true;
    }

    // Two parts of one launch may not see each other's results: what one
    // writes, no other part reads or writes.
    static bool independent(const Part & a, const Part & b) {
        for (const Span & w : a.writes) {
            if (overlaps(w, b.reads) || overlaps(w, b.writes)) {
                return false;
            }
        }
        for (const Span & w : b.writes) {
            if (overlaps(w, a.reads)) {
                return false;
            }
        }
        return true;
    }

    // The attention block's q and k runs (src/arch/qwen3-tts/operations.cpp:
    // 98-104) and the cache copies of k and v (:109-116) as one launch.
    // `a` is a rope run at window positions [p, p + used); its sibling is the
    // next rope run within kSiblingScan positions with the same positions,
    // eps, rope parameters, head size and gain type. The part ending in a
    // copy is k (the cache write); with none, or both, `a` is q. When k's
    // part ends in a copy, the first F32 copy of k's input shape in the scan
    // window that can move up is v's. ggml_build_forward_expand puts the k
    // and v copies before the q path (:106-116), so either part may come
    // first.
    bool match_sibling(size_t p, int used, const Launch & a, Launch & out) {
        const size_t lim   = std::min(order_.size(), p + used + kSiblingScan);
        const bool   a_cpy = is(order_[p + used - 1], SHP_NODE_CPY);
        const Part   pa    = part_of(p, used, order_[p + used - 1]);
        for (size_t p2 = p + used; p2 < lim; ++p2) {
            if (!is(order_[p2], SHP_NODE_RMS_NORM)) {
                continue;
            }
            Launch b;
            int    used_b = 0;
            for (int k : { 5, 4, 3 }) {
                if ((used_b = match_norm(p2, k, b)) != 0) {
                    break;
                }
            }
            if (used_b == 0 || b.kind != SHP_RUN_NORM_MUL_ROPE || !siblings(a, b)) {
                continue;
            }
            const bool   b_cpy = is(order_[p2 + used_b - 1], SHP_NODE_CPY);
            const Part   pb    = part_of(p2, used_b, order_[p2 + used_b - 1]);
            Members      all   = pa.nodes;
            for (int m = 0; m < pb.nodes.n; ++m) {
                all.push(pb.nodes.v[m]);
            }
            if (!independent(pa, pb) || !can_move_up(pb, p, all)) {
                continue;
            }
            const bool     swap = a_cpy && !b_cpy;  // b is q, a is k
            const Launch & q    = swap ? b : a;
            const Launch & k    = swap ? a : b;
            out                 = Launch{};
            out.kind            = SHP_RUN_QK_NORM_ROPE;
            out.x               = q.x;
            out.w               = q.w;
            out.y               = q.y;
            out.x2              = k.x;
            out.w2              = k.w;
            out.y2              = k.y;
            out.b               = a.b;
            out.i0              = a.i0;
            out.f0              = a.f0;
            out.f1              = a.f1;
            out.f2              = a.f2;
            out.first           = order_[p];
            out.last            = std::max(order_[p + used - 1], order_[p2 + used_b - 1]);
            out.count           = used + used_b;
            {
                DryRun dry;
                if (launch_run(*this, out, nullptr) != SHP_OK) {
                    continue;
                }
            }
            std::vector<size_t> taken;
            for (int m = 0; m < used_b; ++m) {
                taken.push_back(p2 + m);
            }
            if (swap ? a_cpy : b_cpy) {
                size_t pv = 0;
                if (find_v_copy(p, used, p2, used_b, *k.x, pa, pb, all, out, pv)) {
                    taken.push_back(pv);
                }
            }
            // the moved-up parts leave the window order, last position first
            std::sort(taken.begin(), taken.end());
            for (size_t t = taken.size(); t-- > 0;) {
                order_.erase(order_.begin() + static_cast<std::ptrdiff_t>(taken[t]));
            }
            return true;
        }
        return false;
    }

    // v's cache copy for a q/k run: a CPY of an F32 tensor of k's input shape
    // into an F32 tensor of that shape, at a window position after p other
    // than the sibling's, that can move up to p next to the other parts. On
    // success `out` becomes the KV launch and *pos_v its window position.
    bool find_v_copy(size_t p, int used, size_t p2, int used_b, const shp_tensor & kx, const Part & pa,
                     const Part & pb, const Members & all, Launch & out, size_t & pos_v) {
        const size_t lim = std::min(order_.size(), p + used + kSiblingScan);
        for (size_t pv = p + used; pv < lim; ++pv) {
            if (pv >= p2 && pv < p2 + used_b) {
                continue;
            }
            const int        c = order_[pv];
            const shp_node & C = nodes_[c];
            if (!is(c, SHP_NODE_CPY) || !f32_of(C.src[0]) || !same_shape(C.src[0], kx) || !f32_of(C.dst) ||
                !same_shape(C.dst, kx)) {
                continue;
            }
            const Part pc   = part_of(pv, 1, c);
            Members    all3 = all;
            all3.push(c);
            if (!independent(pa, pc) || !independent(pb, pc) || !can_move_up(pc, p, all3)) {
                continue;
            }
            Launch kv = out;
            kv.kind   = SHP_RUN_QK_NORM_ROPE_KV;
            kv.x3     = &C.src[0];
            kv.y3     = const_cast<shp_tensor *>(&C.dst);
            kv.last   = std::max(out.last, c);
            kv.count  = out.count + 1;
            DryRun dry;
            if (launch_run(*this, kv, nullptr) != SHP_OK) {
                continue;
            }
            out   = kv;
            pos_v = pv;
            return true;
        }
        return false;
    }

    // Two rope runs one launch can take: the same positions tensor, eps,
    // n_dims, base and scale (bit for bit), head size and token count, and
    // gains of one type.
    static bool siblings(const Launch & a, const Launch & b) {
        auto bits = [](float f) {
            uint32_t u;
            std::memcpy(&u, &f, sizeof(u));
            return u;
        };
        return same_tensor(*a.b, *b.b) && a.i0 == b.i0 && bits(a.f0) == bits(b.f0) && bits(a.f1) == bits(b.f1) &&
               bits(a.f2) == bits(b.f2) && a.x->ne[0] == b.x->ne[0] && a.x->ne[2] == b.x->ne[2] &&
               a.w->type == b.w->type;
    }

    const shp_node *              nodes_;
    int                           n_;
    std::vector<int> order_;
    std::vector<int> cstart_;
    std::vector<int> cons_;

    int readers(int j) const { return cstart_[j + 1] - cstart_[j]; }

    // Node index at window position p + k, or -1 past the end.
    int at(size_t p, int k) const { return p + k < order_.size() ? order_[p + k] : -1; }

    // The window order_[p, p + members.n) holds exactly `members` (distinct
    // node indices).
    bool window_is(size_t p, const Members & members) const {
        if (p + members.n > order_.size()) {
            return false;
        }
        for (int k = 0; k < members.n; ++k) {
            if (!members.has(order_[p + k])) {
                return false;
            }
        }
        return true;
    }

    // j's result may go unwritten: not an output, read by no later split and
    // by no node of the list outside `members`.
    bool internal(int j, const Members & members) const {
        if (nodes_[j].flags & SHP_NODE_FLAG_OUTPUT) {
            return false;
        }
        if (readers(j) == 0 || nodes_[j].uses > readers(j)) {
            return false;
        }
        for (int c = cstart_[j]; c < cstart_[j + 1]; ++c) {
            if (!members.has(cons_[c])) {
                return false;
            }
        }
        return true;
    }

    // internal(), with view nodes between j and its readers looked through: a
    // view (NOP) reader counts when it is no output, no later split reads it,
    // and its own readers are members (or views of the same kind).
    bool internal_v(int j, const Members & members, int depth = 0) const {
        if (depth > 8 || (nodes_[j].flags & SHP_NODE_FLAG_OUTPUT) || readers(j) == 0 ||
            nodes_[j].uses > readers(j)) {
            return false;
        }
        for (int c = cstart_[j]; c < cstart_[j + 1]; ++c) {
            const int r = cons_[c];
            if (members.has(r)) {
                continue;
            }
            if (nodes_[r].op != SHP_NODE_NOP || !internal_v(r, members, depth + 1)) {
                return false;
            }
        }
        return true;
    }

    // j's result is read outside `members` (or is an output): it must be written.
    bool needed_outside(int j, const Members & members) const {
        return (nodes_[j].flags & SHP_NODE_FLAG_OUTPUT) || !internal(j, members);
    }

    bool is(int j, int op) const { return j >= 0 && nodes_[j].op == op; }

    int src(int j, int k) const { return nodes_[j].src_node[k]; }

    // The longest run that starts at window position p (0: none). Runs are
    // tried by the op of their first node.
    int match(size_t p, Launch & l) const {
        int used = 0;
        switch (nodes_[order_[p]].op) {
            case SHP_NODE_GET_ROWS:
                return match_gather_sum(p, l);
            case SHP_NODE_MUL:
            case SHP_NODE_EXP:
            case SHP_NODE_SCALE:
                for (int k : { 8, 6, 5 }) {
                    if ((used = match_snake(p, k, l)) != 0) {
                        return used;
                    }
                }
                return match_mul_sum_rows(p, l);
            case SHP_NODE_ADD:
                if ((used = match_transpose_bias(p, l)) != 0) {
                    return used;
                }
                for (int k : { 4, 3 }) {
                    if ((used = match_add_norm(p, k, l)) != 0) {
                        return used;
                    }
                }
                for (int k = 2 + 7; k >= 3; --k) {
                    if ((used = match_add_scale_leaky(p, k, l)) != 0) {
                        return used;
                    }
                }
                return match_add_leaky(p, l);
            case SHP_NODE_RMS_NORM:
                for (int k : { 5, 4, 3, 2 }) {
                    if ((used = match_norm(p, k, l)) != 0) {
                        return used;
                    }
                }
                return 0;
            case SHP_NODE_SILU:
                return match_silu_mul(p, l);
            case SHP_NODE_DIAG_MASK_INF:
                return match_causal_soft_max(p, l);
            case SHP_NODE_CPY:
                if ((used = match_transpose_bias(p, l)) != 0 || (used = match_cont_tail(p, l)) != 0 ||
                    (used = match_cont_im2col(p, l)) != 0) {
                    return used;
                }
                return match_view_binary(p, l);
            default:
                return 0;
        }
    }

    // GET_ROWS, then (GET_ROWS, ADD(acc, rows)) per further group: the tables
    // share a type and row length, the ids are the columns of one contiguous
    // I32 [frames, groups] tensor (consecutive views, code-predictor.cpp:99).
    int match_gather_sum(size_t p, Launch & l) const {
        const int g0 = at(p, 0);
        if (!is(g0, SHP_NODE_GET_ROWS) || !single_ok(nodes_[g0])) {
            return 0;
        }
        const shp_tensor & t0   = nodes_[g0].src[0];
        const shp_tensor & ids0 = nodes_[g0].src[1];
        const int64_t      fr   = ids0.ne[0];
        if (ids0.ne[1] != 1 || ids0.ne[2] != 1 || !contiguous(ids0) || !contiguous(nodes_[g0].dst)) {
            return 0;
        }
        Members members{ g0 };
        int     acc    = g0;
        int     groups = 1;
        int     best   = 0;
        int     last   = -1;
        while (groups < 64) {
            const int gr = at(p, 2 * groups - 1);
            const int ad = at(p, 2 * groups);
            if (!is(gr, SHP_NODE_GET_ROWS) || !is(ad, SHP_NODE_ADD)) {
                break;
            }
            const shp_node & G = nodes_[gr];
            const shp_node & A = nodes_[ad];
            const bool order_ok = (src(ad, 0) == acc && src(ad, 1) == gr) || (src(ad, 1) == acc && src(ad, 0) == gr);
            const auto & ids    = G.src[1];
            const bool   ids_ok = well_formed(&ids) && ids.type == SHP_TYPE_I32 && ids.ne[0] == fr && ids.ne[1] == 1 &&
                                ids.ne[2] == 1 && ids.ne[3] == 1 &&
                                static_cast<const char *>(ids.data) ==
                                    static_cast<const char *>(ids0.data) + static_cast<size_t>(groups) * fr * 4;
            const bool tab_ok = well_formed(&G.src[0]) && G.src[0].type == t0.type && G.src[0].ne[0] == t0.ne[0] &&
                                single_ok(G);
            if (!order_ok || !ids_ok || !tab_ok || !f32_of(A.dst) || !same_shape(A.dst, nodes_[g0].dst)) {
                break;
            }
            members.push(gr);
            members.push(ad);
            acc = ad;
            ++groups;
            // Every result before the last add is read only inside the run.
            bool ok = true;
            for (int m = 0; m + 1 < members.n; ++m) {
                ok = ok && internal(members.v[m], members);
            }
            if (ok) {
                best = groups;
                last = ad;
            }
        }
        if (best < 2) {
            return 0;
        }
        l.kind = SHP_RUN_GATHER_SUM;
        l.terms.clear();
        l.terms.push_back(t0);
        for (int g = 1; g < best; ++g) {
            l.terms.push_back(nodes_[members.v[2 * g - 1]].src[0]);
        }
        l.codes       = ids0;
        l.codes.ne[1] = best;
        l.codes.nb[1] = static_cast<size_t>(fr) * 4;
        l.codes.nb[2] = l.codes.nb[1] * best;
        l.codes.nb[3] = l.codes.nb[2];
        l.y           = const_cast<shp_tensor *>(&nodes_[last].dst);
        return 2 * best - 1;
    }

    // The Snake family, k = 5 (Snake), 6 (guarded), 8 (SnakeBeta):
    //   ADD(x, DIV(SQ(SIN(MUL(x, al))), den)) with SQ = MUL(s, s) or SQR(s);
    //   Snake: den = al; guarded: den = SCALE(al, 1, 1e-9);
    //   SnakeBeta: al = EXP(la), den = SCALE(EXP(lb), 1, 1e-9).
    int match_snake(size_t p, int k, Launch & l) const {
        const int ad = at(p, k - 1);
        if (!is(ad, SHP_NODE_ADD)) {
            return 0;
        }
        const shp_node & A  = nodes_[ad];
        const int        dv = src(ad, 1);
        if (!is(dv, SHP_NODE_DIV)) {
            return 0;
        }
        const int sq = src(dv, 0);
        int       sn = -1;
        if (is(sq, SHP_NODE_MUL) && src(sq, 0) >= 0 && src(sq, 0) == src(sq, 1)) {
            sn = src(sq, 0);
        } else if (is(sq, SHP_NODE_SQR)) {
            sn = src(sq, 0);
        }
        if (!is(sn, SHP_NODE_SIN)) {
            return 0;
        }
        const int ml = src(sn, 0);
        if (!is(ml, SHP_NODE_MUL)) {
            return 0;
        }
        const shp_node & M = nodes_[ml];
        const shp_tensor & x = A.src[0];
        if (!f32_of(x) || !same_tensor(M.src[0], x) || !f32_of(A.dst) || !same_shape(A.dst, x)) {
            return 0;
        }
        const int64_t C = x.ne[0];
        const int     den = src(dv, 1);
        Members members{ ml, sn, sq, dv, ad };
        auto curve_ok = [C](const shp_tensor & c) {
            return well_formed(&c) && c.type == SHP_TYPE_F32 && one_row_of(c, C);
        };
        auto guard_ok = [&](int j) {
            return is(j, SHP_NODE_SCALE) && fparam(nodes_[j], 0) == 1.0f && fparam(nodes_[j], 1) == 1e-9f;
        };
        int kind;
        if (k == 5) {
            if (den != -1 && src(ml, 1) != den) {
                return 0;
            }
            if (!curve_ok(M.src[1]) || !same_tensor(nodes_[dv].src[1], M.src[1])) {
                return 0;
            }
            kind = SHP_RUN_SNAKE;
            l.w  = &M.src[1];
        } else if (k == 6) {
            if (!guard_ok(den) || !curve_ok(M.src[1]) || !same_tensor(nodes_[den].src[0], M.src[1])) {
                return 0;
            }
            members.push(den);
            kind = SHP_RUN_SNAKE_GUARDED;
            l.w  = &M.src[1];
        } else {
            const int ea = src(ml, 1);
            if (!is(ea, SHP_NODE_EXP) || !guard_ok(den)) {
                return 0;
            }
            const int eb = src(den, 0);
            if (!is(eb, SHP_NODE_EXP) || eb == ea || !curve_ok(nodes_[ea].src[0]) || !curve_ok(nodes_[eb].src[0])) {
                return 0;
            }
            members.push(den);
            members.push(ea);
            members.push(eb);
            kind = SHP_RUN_SNAKE_BETA;
            l.w  = &nodes_[ea].src[0];
            l.c1 = &nodes_[eb].src[0];
        }
        if (members.n != k || !window_is(p, members)) {
            return 0;
        }
        for (int m = 0; m < members.n; ++m) {
            if (members.v[m] != ad && !internal(members.v[m], members)) {
                return 0;
            }
        }
        l.kind = kind;
        l.x    = &A.src[0];
        l.y    = const_cast<shp_tensor *>(&A.dst);
        return k;
    }

    // MUL(n, w) whose n is the RMS_NORM `nrm`. When `cast` (a window node, or
    // -1) produced w, the gain is that CPY's source (the as_f32 cast folded
    // in) and `cast` is returned; otherwise w itself must be an F32 gain and
    // -2 is returned. -1: not a gain multiply.
    int gain_of(int mul, int nrm, int cast, const shp_tensor *& w, int64_t ne0) const {
        const shp_node & M = nodes_[mul];
        if (src(mul, 0) != nrm) {
            return -1;
        }
        if (cast >= 0) {
            if (src(mul, 1) != cast || !is(cast, SHP_NODE_CPY)) {
                return -1;
            }
            const shp_node & Cp = nodes_[cast];
            if (!gain_vector(Cp.src[0], ne0) || !f32_of(Cp.dst) || !same_shape(Cp.src[0], Cp.dst)) {
                return -1;
            }
            w = &Cp.src[0];
            return cast;
        }
        if (!gain_vector(M.src[1], ne0) || M.src[1].type != SHP_TYPE_F32) {
            return -1;
        }
        w = &M.src[1];
        return -2;
    }

    // RMS_NORM [CPY] MUL [ROPE [CPY]], k nodes.
    int match_norm(size_t p, int k, Launch & l) const {
        const int nrm = at(p, 0);
        if (!is(nrm, SHP_NODE_RMS_NORM) || at(p, k - 1) < 0) {
            return 0;
        }
        const shp_node & N = nodes_[nrm];
        if (!unary_ok(N) || !(fparam(N, 0) >= 0.0f)) {
            return 0;
        }
        const int64_t ne0 = N.src[0].ne[0];
        // Find the MUL: position 1 or 2.
        for (int mpos : { 1, 2 }) {
            const int mul = at(p, mpos);
            if (!is(mul, SHP_NODE_MUL) || mpos >= k) {
                continue;
            }
            const shp_tensor * w    = nullptr;
            const int          cast = gain_of(mul, nrm, mpos == 2 ? at(p, 1) : -1, w, ne0);
            if (cast == -1) {
                continue;
            }
            if (!f32_of(nodes_[mul].dst) || !same_shape(nodes_[mul].dst, N.src[0])) {
                continue;
            }
            Members members{ nrm, mul };
            if (cast >= 0) {
                members.push(cast);
            }
            const int rest = k - members.n;
            int       rope = -1, cp = -1;
            if (rest >= 1) {
                rope = at(p, mpos + 1);
                if (!is(rope, SHP_NODE_ROPE) || src(rope, 0) != mul || !rope_params_ok(nodes_[rope]) ||
                    fparam(nodes_[rope], 8) != 1.0f) {
                    continue;
                }
                members.push(rope);
            }
            if (rest == 2) {
                cp = at(p, mpos + 2);
                if (!is(cp, SHP_NODE_CPY) || src(cp, 0) != rope || !f32_of(nodes_[cp].dst) ||
                    !same_shape(nodes_[cp].dst, nodes_[rope].dst)) {
                    continue;
                }
                members.push(cp);
            }
            if (rest > 2 || !window_is(p, members)) {
                continue;
            }
            const int sink = cp >= 0 ? cp : (rope >= 0 ? rope : mul);
            bool      ok   = true;
            for (int m = 0; m < members.n; ++m) {
                ok = ok && (members.v[m] == sink || internal(members.v[m], members));
            }
            if (!ok) {
                continue;
            }
            l.x  = &N.src[0];
            l.w  = w;
            l.f0 = fparam(N, 0);
            l.y  = const_cast<shp_tensor *>(&nodes_[sink].dst);
            if (rope >= 0) {
                const shp_node & R = nodes_[rope];
                l.kind             = SHP_RUN_NORM_MUL_ROPE;
                l.b                = &R.src[1];
                l.i0               = R.op_params[1];
                l.f1               = fparam(R, 5);
                l.f2               = fparam(R, 6);
            } else {
                l.kind = SHP_RUN_NORM_MUL;
            }
            return k;
        }
        return 0;
    }

    // ADD RMS_NORM [CPY] MUL, k nodes; the sum is written when read elsewhere.
    int match_add_norm(size_t p, int k, Launch & l) const {
        const int ad  = at(p, 0);
        const int nrm = at(p, 1);
        const int mul = at(p, k - 1);
        if (!is(ad, SHP_NODE_ADD) || !is(nrm, SHP_NODE_RMS_NORM) || !is(mul, SHP_NODE_MUL) || src(nrm, 0) != ad) {
            return 0;
        }
        const shp_node & A = nodes_[ad];
        const shp_node & N = nodes_[nrm];
        if (!f32_of(A.src[0]) || !f32_of(A.src[1]) || !same_shape(A.src[0], A.src[1]) || !f32_of(A.dst) ||
            !same_shape(A.src[0], A.dst) || !unary_ok(N) || !(fparam(N, 0) >= 0.0f)) {
            return 0;
        }
        const shp_tensor * w    = nullptr;
        const int          cast = gain_of(mul, nrm, k == 4 ? at(p, 2) : -1, w, A.dst.ne[0]);
        if (cast == -1) {
            return 0;
        }
        if (!f32_of(nodes_[mul].dst) || !same_shape(nodes_[mul].dst, A.dst)) {
            return 0;
        }
        Members members{ ad, nrm, mul };
        if (cast >= 0) {
            members.push(cast);
        }
        if (!window_is(p, members) || !internal(nrm, members) || (cast >= 0 && !internal(cast, members))) {
            return 0;
        }
        l.kind = SHP_RUN_ADD_NORM_MUL;
        l.x    = &A.src[0];
        l.b    = &A.src[1];
        l.w    = w;
        l.f0   = fparam(N, 0);
        l.sum  = needed_outside(ad, members) ? const_cast<shp_tensor *>(&A.dst) : nullptr;
        l.y    = const_cast<shp_tensor *>(&nodes_[mul].dst);
        return k;
    }

    // ADD x (k-2), SCALE(b = 0), LEAKY_RELU: the terms in add order.
    int match_add_scale_leaky(size_t p, int k, Launch & l) const {
        const int nadd = k - 2;
        const int sc   = at(p, k - 2);
        const int lk   = at(p, k - 1);
        if (nadd < 1 || nadd > 7 || !is(sc, SHP_NODE_SCALE) || !is(lk, SHP_NODE_LEAKY_RELU) || src(lk, 0) != sc ||
            fparam(nodes_[sc], 1) != 0.0f) {
            return 0;
        }
        Members                 members;
        std::vector<shp_tensor> terms;
        int                     acc = -1;
        for (int a = 0; a < nadd; ++a) {
            const int ad = at(p, a);
            if (!is(ad, SHP_NODE_ADD)) {
                return 0;
            }
            const shp_node & A = nodes_[ad];
            if (!f32_of(A.src[0]) || !f32_of(A.src[1]) || !same_shape(A.src[0], A.src[1]) || !f32_of(A.dst) ||
                !same_shape(A.dst, A.src[0]) || !contiguous(A.src[0]) || !contiguous(A.src[1])) {
                return 0;
            }
            if (a == 0) {
                terms.push_back(A.src[0]);
                terms.push_back(A.src[1]);
            } else if (src(ad, 0) == acc) {
                terms.push_back(A.src[1]);
            } else if (src(ad, 1) == acc) {
                terms.push_back(A.src[0]);
            } else {
                return 0;
            }
            acc = ad;
            members.push(ad);
        }
        if (src(sc, 0) != acc) {
            return 0;
        }
        members.push(sc);
        members.push(lk);
        for (int a = 0; a < nadd; ++a) {
            if (!internal(members.v[a], members)) {
                return 0;
            }
        }
        const shp_node & S = nodes_[sc];
        const shp_node & L = nodes_[lk];
        if (!f32_of(L.dst) || !same_shape(L.dst, S.dst) || !contiguous(L.dst) || !contiguous(S.dst)) {
            return 0;
        }
        l.kind  = SHP_RUN_ADD_SCALE_LEAKY;
        l.terms = terms;
        l.f0    = fparam(S, 0);
        l.f1    = fparam(L, 0);
        l.sum   = needed_outside(sc, members) ? const_cast<shp_tensor *>(&S.dst) : nullptr;
        l.y     = const_cast<shp_tensor *>(&L.dst);
        return k;
    }

    int match_add_leaky(size_t p, Launch & l) const {
        const int ad = at(p, 0);
        const int lk = at(p, 1);
        if (!is(ad, SHP_NODE_ADD) || !is(lk, SHP_NODE_LEAKY_RELU) || src(lk, 0) != ad) {
            return 0;
        }
        const shp_node & A = nodes_[ad];
        const shp_node & L = nodes_[lk];
        if (!f32_of(A.src[0]) || !f32_of(A.src[1]) || !same_shape(A.src[0], A.src[1]) || !f32_of(A.dst) ||
            !same_shape(A.dst, A.src[0]) || !unary_ok(L)) {
            return 0;
        }
        const Members members{ ad, lk };
        l.kind = SHP_RUN_ADD_LEAKY;
        l.x    = &A.src[0];
        l.b    = &A.src[1];
        l.f0   = fparam(L, 0);
        l.sum  = needed_outside(ad, members) ? const_cast<shp_tensor *>(&A.dst) : nullptr;
        l.y    = const_cast<shp_tensor *>(&L.dst);
        return 2;
    }

    // The tail of the time-major vocoder convolution (vits/waveform-decoder.cpp:
    // 111,118-121 and what follows it, :146-150): CPY of the GEMM output's
    // transposed view, ADD(copy, bias) with the bias as src1, then
    // optionally ADD(sum, residual) (either operand order) and LEAKY_RELU of
    // the last sum. The copy's result is never written and must be read by
    // the bias add alone; the biased value is written only when no residual
    // add follows and something outside reads it (as the run's sum).
    int match_cont_tail(size_t p, Launch & l) const {
        const int cp = at(p, 0);
        const int ab = at(p, 1);
        if (!is(cp, SHP_NODE_CPY) || !is(ab, SHP_NODE_ADD) || src(ab, 0) != cp || src(ab, 1) == cp) {
            return 0;
        }
        const shp_node & C = nodes_[cp];
        const shp_node & A = nodes_[ab];
        if (f32_strided_view_dim(&C.src[0]) == 0 || !f32_of(C.dst) || !same_shape(C.src[0], C.dst) ||
            !f32_of(A.dst) || !same_shape(A.dst, C.dst) || !f32_of(A.src[1])) {
            return 0;
        }
        // optional residual add at position 2
        const int ar    = at(p, 2);
        int       other = -1;
        if (is(ar, SHP_NODE_ADD) && (src(ar, 0) == ab) != (src(ar, 1) == ab)) {
            other               = src(ar, 0) == ab ? 1 : 0;
            const shp_node & R2 = nodes_[ar];
            if (!f32_of(R2.src[other]) || !same_shape(R2.src[other], A.dst) || !f32_of(R2.dst) ||
                !same_shape(R2.dst, A.dst)) {
                other = -1;
            }
        }
        for (int with_r = other >= 0 ? 1 : 0; with_r >= 0; --with_r) {
            const int last = with_r ? ar : ab;
            const int lk   = at(p, with_r ? 3 : 2);
            for (int with_l = (is(lk, SHP_NODE_LEAKY_RELU) && src(lk, 0) == last && unary_ok(nodes_[lk])) ? 1 : 0;
                 with_l >= 0; --with_l) {
                Members members{ cp, ab };
                if (with_r) {
                    members.push(ar);
                }
                if (with_l) {
                    members.push(lk);
                }
                if (!internal(cp, members) || (with_r && !internal(ab, members))) {
                    continue;
                }
                l.kind = SHP_RUN_CONT_ADD_LEAKY;
                l.x    = &C.src[0];
                l.b    = &A.src[1];
                l.x3   = with_r ? &nodes_[ar].src[other] : nullptr;
                l.i0   = with_l;
                l.f0   = with_l ? fparam(nodes_[lk], 0) : 0.0f;
                l.sum  = with_l && needed_outside(last, members) ? const_cast<shp_tensor *>(&nodes_[last].dst) : nullptr;
                l.y    = const_cast<shp_tensor *>(&nodes_[with_l ? lk : last].dst);
                return members.n;
            }
        }
        return 0;
    }

    // t is exactly ggml_transpose(s): s's data with dims 0 and 1 swapped.
    // (A stride is compared only where its extent is above 1: it is never
    // used otherwise.)
    static bool is_transpose_of(const shp_tensor & t, const shp_tensor & s) {
        const auto same = [&](int dt, int ds) { return t.ne[dt] == 1 || t.nb[dt] == s.nb[ds]; };
        return t.data == s.data && t.type == s.type && t.ne[0] == s.ne[1] && t.ne[1] == s.ne[0] &&
               t.ne[2] == s.ne[2] && t.ne[3] == s.ne[3] && same(0, 1) && same(1, 0) && same(2, 2) && same(3, 3);
    }

    // The channel-major convolutions' tails (qwen3-tts/codec.cpp), as one
    // transposing copy with the channel bias added per destination column:
    //  (a) [CPY(row-contiguous view v) ->] ADD(v, b [1, C]) -> CPY(transpose
    //      of the sum) (the transposed convolution's crop, bias and return,
    //      :179-181): y = transpose(v) + b read as one row of C;
    //  (b) CPY(transposed view t) -> CPY(its first rows) -> ADD(crop, b [C])
    //      (the depthwise convolution's return to channel-major, crop and
    //      bias, :134-140): y = the first rows of the transposing copy + b.
    // Each add is exact per element, so adding before or after the transpose
    // gives the same bits.
    int match_transpose_bias(size_t p, Launch & l) const {
        const int n0 = at(p, 0), n1 = at(p, 1), n2 = at(p, 2);
        // (b)
        if (is(n0, SHP_NODE_CPY) && is(n1, SHP_NODE_CPY) && is(n2, SHP_NODE_ADD) && producer(n1, 0) == n0 &&
            src(n2, 0) == n1 && src(n2, 1) != n1) {
            const shp_node & T = nodes_[n0];
            const shp_node & K = nodes_[n1];
            const shp_node & A = nodes_[n2];
            const shp_tensor & crop = K.src[0];
            const Members members{ n0, n1, n2 };
            if (f32_strided_view_dim(&T.src[0]) != 0 && f32_of(T.dst) && same_shape(T.src[0], T.dst) &&
                f32_of(crop) && crop.data == T.dst.data && crop.ne[0] == T.dst.ne[0] && crop.ne[1] <= T.dst.ne[1] &&
                crop.ne[2] == T.dst.ne[2] && crop.ne[3] == T.dst.ne[3] &&
                (crop.ne[1] == 1 || crop.nb[1] == T.dst.nb[1]) && (crop.ne[2] == 1 || crop.nb[2] == T.dst.nb[2]) &&
                (crop.ne[3] == 1 || crop.nb[3] == T.dst.nb[3]) && f32_of(K.dst) &&
                same_shape(K.dst, crop) && f32_of(A.dst) && same_shape(A.dst, crop) && internal_v(n0, members) &&
                internal(n1, members)) {
                l      = Launch{};
                l.kind = SHP_RUN_CONT_ADD_LEAKY;
                l.xv   = T.src[0];
                l.xv.ne[1] = crop.ne[1];  // only the rows the crop keeps
                l.own_x    = true;
                l.b        = &A.src[1];
                l.y        = const_cast<shp_tensor *>(&A.dst);
                return 3;
            }
        }
        // (a), with or without the crop's copy in front
        const bool crop = is(n0, SHP_NODE_CPY);
        const int  ad = crop ? n1 : n0, cp = crop ? n2 : n1;
        if (!is(ad, SHP_NODE_ADD) || !is(cp, SHP_NODE_CPY) || (crop && (src(ad, 0) != n0 || src(ad, 1) == n0)) ||
            producer(cp, 0) != ad) {
            return 0;
        }
        const shp_node & A = nodes_[ad];
        const shp_node & C = nodes_[cp];
        const shp_tensor & v = crop ? nodes_[n0].src[0] : A.src[0];
        const shp_tensor & b = A.src[1];
        Members members{ ad, cp };
        if (crop) {
            members.push(n0);
        }
        if (!f32_of(v) || !f32_of(A.dst) || !same_shape(v, A.dst) || (crop && !same_shape(nodes_[n0].dst, v)) ||
            !is_transpose_of(C.src[0], A.dst) || !f32_of(C.dst) || !same_shape(C.dst, C.src[0]) ||
            !internal_v(ad, members) || (crop && !internal(n0, members)) || !well_formed(&b) ||
            b.type != SHP_TYPE_F32 || b.ne[0] != 1 || b.ne[1] != v.ne[1] || b.ne[2] != 1 || b.ne[3] != 1 ||
            b.nb[1] != 4 || v.ne[2] != 1 || v.ne[3] != 1) {
            return 0;
        }
        l       = Launch{};
        l.kind  = SHP_RUN_CONT_ADD_LEAKY;
        l.xv    = v;  // transpose(v): dims 0 and 1 swapped
        l.xv.ne[0] = v.ne[1];
        l.xv.ne[1] = v.ne[0];
        l.xv.nb[0] = v.nb[1];
        l.xv.nb[1] = v.nb[0];
        l.own_x    = true;
        l.bv       = b;  // [1, C] read as one row of C
        l.bv.ne[0] = b.ne[1];
        l.bv.ne[1] = 1;
        l.bv.nb[0] = b.nb[1];
        l.own_b    = true;
        l.y        = const_cast<shp_tensor *>(&C.dst);
        return members.n;
    }

    // CPY of a row-contiguous F32 view into a tensor of its shape, read only
    // by an ADD, MUL or DIV as src0: the op reads the view in place of the
    // copy, which is never written (the causal convolutions' crop, then their
    // channel bias: qwen3-tts/codec.cpp:64-71,100-104,137-140). The copy is
    // exact, so the result is the same bits.
    int match_view_binary(size_t p, Launch & l) const {
        const int cp = at(p, 0);
        const int op = at(p, 1);
        if (!is(cp, SHP_NODE_CPY) || !(is(op, SHP_NODE_ADD) || is(op, SHP_NODE_MUL) || is(op, SHP_NODE_DIV)) ||
            src(op, 0) != cp || src(op, 1) == cp) {
            return 0;
        }
        const shp_node & C = nodes_[cp];
        const shp_node & B = nodes_[op];
        // The op's result may sit in memory the copy's source gave up (the
        // allocator reuses it once the copy has run): reading the view while
        // writing it in another row stride would go wrong, so any overlap
        // leaves the nodes apart.
        if (!f32_of(C.src[0]) || !f32_of(C.dst) || !same_shape(C.src[0], C.dst) || !internal(cp, Members{ cp, op }) ||
            spans_overlap(C.src[0], B.dst)) {
            return 0;
        }
        shp_node n = B;  // the op with the view as src0
        n.src[0]   = C.src[0];
        if (!binary_ok(n)) {
            return 0;
        }
        l.kind = SHP_RUN_VIEW_BINARY;
        l.i0   = B.op;
        l.x    = &C.src[0];
        l.b    = &B.src[1];
        l.y    = const_cast<shp_tensor *>(&B.dst);
        return 2;
    }

    // CPY of a transposed F32 view into a contiguous tensor -- the causal
    // convolution's ggml_cont(ggml_transpose(x)) of a channel-major activation
    // -- read only by IM2COL as its input, directly or through view nodes that
    // add or drop extents of 1 (qwen3-tts/codec.cpp:94-96): shp_im2col reads
    // the activation through the transposed view, and the copy is never
    // written. Taken when that view has its channels contiguous, which the
    // kernel loads coalesced; the depthwise form (channels as batch entries,
    // :124-129) keeps its copy.
    int match_cont_im2col(size_t p, Launch & l) const {
        const int cp = at(p, 0);
        const int im = at(p, 1);
        if (!is(cp, SHP_NODE_CPY) || !is(im, SHP_NODE_IM2COL) || producer(im, 1) != cp || producer(im, 0) == cp) {
            return 0;
        }
        const shp_node &   C = nodes_[cp];
        const shp_node &   I = nodes_[im];
        const shp_tensor & s = C.src[0];
        const shp_tensor & b = I.src[1];
        if (f32_strided_view_dim(&s) == 0 || !f32_of(C.dst) || !same_shape(s, C.dst) || !contiguous(C.dst) ||
            !f32_of(b) || b.data != C.dst.data || !contiguous(b) || !internal_v(cp, Members{ cp, im })) {
            return 0;
        }
        // b is the copy's result with extents of 1 added or dropped: map each
        // of its dimensions of extent > 1 to the source's, in order
        shp_tensor v = b;
        int        sd[4], bd[4], ns = 0, nb = 0;
        for (int d = 0; d < 4; ++d) {
            if (s.ne[d] > 1) {
                sd[ns++] = d;
            }
            if (b.ne[d] > 1) {
                bd[nb++] = d;
            }
        }
        if (ns != nb) {
            return 0;
        }
        for (int i = 0; i < ns; ++i) {
            if (s.ne[sd[i]] != b.ne[bd[i]]) {
                return 0;
            }
            v.nb[bd[i]] = s.nb[sd[i]];
        }
        v.data = s.data;
        if (v.nb[1] != 4 || v.nb[0] == 4 || v.ne[1] < 2) {
            return 0;
        }
        l       = Launch{};
        l.kind  = SHP_RUN_CONT_IM2COL;
        l.xv    = v;
        l.own_x = true;
        l.w     = &I.src[0];
        l.i0    = I.op_params[0];  // s0
        l.i1    = I.op_params[2];  // p0
        l.i2    = I.op_params[4];  // d0
        l.y     = const_cast<shp_tensor *>(&I.dst);
        return 2;
    }

    // DIAG_MASK_INF then a maskless SOFT_MAX of its result with a positive
    // finite scale, the masked scores read nowhere else.
    int match_causal_soft_max(size_t p, Launch & l) const {
        const int dm = at(p, 0);
        const int sm = at(p, 1);
        if (!is(dm, SHP_NODE_DIAG_MASK_INF) || !is(sm, SHP_NODE_SOFT_MAX) || src(sm, 0) != dm) {
            return 0;
        }
        const shp_node & D = nodes_[dm];
        const shp_node & M = nodes_[sm];
        const float      scale = fparam(M, 0);
        if (!single_ok(D) || !single_ok(M) || present(M.src[1]) || !(scale > 0.0f) || !(scale < INFINITY) ||
            !internal(dm, Members{ dm, sm })) {
            return 0;
        }
        l.kind = SHP_RUN_DIAG_MASK_SOFT_MAX;
        l.x    = &D.src[0];
        l.i0   = D.op_params[0];
        l.f0   = scale;
        l.y    = const_cast<shp_tensor *>(&M.dst);
        return 2;
    }

    // MUL(x, w) then SUM_ROWS of the product, the product read nowhere else:
    // x and w of one shape (the attention-weighted sums of the speaker
    // encoder's pooling).
    int match_mul_sum_rows(size_t p, Launch & l) const {
        const int mu = at(p, 0);
        const int sr = at(p, 1);
        if (!is(mu, SHP_NODE_MUL) || !is(sr, SHP_NODE_SUM_ROWS) || src(sr, 0) != mu) {
            return 0;
        }
        const shp_node & M = nodes_[mu];
        const shp_node & S = nodes_[sr];
        if (!f32_of(M.src[0]) || !f32_of(M.src[1]) || !same_shape(M.src[0], M.src[1]) || !f32_of(M.dst) ||
            !same_shape(M.dst, M.src[0]) || !single_ok(S) || !internal(mu, Members{ mu, sr })) {
            return 0;
        }
        l.kind = SHP_RUN_MUL_SUM_ROWS;
        l.x    = &M.src[0];
        l.b    = &M.src[1];
        l.y    = const_cast<shp_tensor *>(&S.dst);
        return 2;
    }

    // SILU(g) then MUL(silu, u) (either operand order: the product commutes).
    int match_silu_mul(size_t p, Launch & l) const {
        const int si = at(p, 0);
        const int mu = at(p, 1);
        if (!is(si, SHP_NODE_SILU) || !is(mu, SHP_NODE_MUL)) {
            return 0;
        }
        const shp_node & M = nodes_[mu];
        int              other;
        if (src(mu, 0) == si && src(mu, 1) != si) {
            other = 1;
        } else if (src(mu, 1) == si && src(mu, 0) != si) {
            other = 0;
        } else {
            return 0;
        }
        const shp_node & S = nodes_[si];
        if (!unary_ok(S) || !f32_of(M.src[other]) || !same_shape(M.src[other], S.dst) || !f32_of(M.dst) ||
            !same_shape(M.dst, S.dst) || !internal(si, Members{ si, mu })) {
            return 0;
        }
        l.kind = SHP_RUN_SILU_MUL;
        l.x    = &S.src[0];
        l.b    = &M.src[other];
        l.y    = const_cast<shp_tensor *>(&M.dst);
        return 2;
    }
};

shp_status_t launch_single(const shp_node & n, shp_stream_t st) {
    shp_tensor * y = const_cast<shp_tensor *>(&n.dst);
    switch (n.op) {
        case SHP_NODE_NOP:
            return SHP_OK;
        case SHP_NODE_ADD:
            return shp_add(&n.src[0], &n.src[1], y, st);
        case SHP_NODE_MUL:
            return shp_mul(&n.src[0], &n.src[1], y, st);
        case SHP_NODE_DIV:
            return shp_div(&n.src[0], &n.src[1], y, st);
        case SHP_NODE_SQR:
            return shp_sqr(&n.src[0], y, st);
        case SHP_NODE_SIN:
            return shp_sin(&n.src[0], y, st);
        case SHP_NODE_SCALE:
            return shp_scale_bias(&n.src[0], fparam(n, 0), fparam(n, 1), y, st);
        case SHP_NODE_CPY:
            return shp_cpy(&n.src[0], y, st);
        case SHP_NODE_GET_ROWS:
            return shp_get_rows(&n.src[0], &n.src[1], y, st);
        case SHP_NODE_RMS_NORM:
            return shp_rms_norm_mul(&n.src[0], nullptr, fparam(n, 0), y, st);
        case SHP_NODE_SOFT_MAX:
            return shp_soft_max_ext(&n.src[0], present(n.src[1]) ? &n.src[1] : nullptr, fparam(n, 0), fparam(n, 1), y,
                                    st);
        case SHP_NODE_ROPE:
            return shp_rope_ext(&n.src[0], &n.src[1], n.op_params[1], n.op_params[2], fparam(n, 5), fparam(n, 6),
                                fparam(n, 7), fparam(n, 8), y, st);
        case SHP_NODE_LEAKY_RELU:
            return shp_add_leaky_relu(&n.src[0], nullptr, fparam(n, 0), nullptr, y, st);
        case SHP_NODE_SILU:
            return shp_swiglu(&n.src[0], nullptr, y, st);
        case SHP_NODE_EXP:
            return shp_exp(&n.src[0], y, st);
        case SHP_NODE_GLU_SWIGLU:
            if (present(n.src[1])) {
                const bool swapped = n.op_params[1] != 0;
                return shp_swiglu(swapped ? &n.src[1] : &n.src[0], swapped ? &n.src[0] : &n.src[1], y, st);
            }
            return shp_glu_swiglu(&n.src[0], n.op_params[1], y, st);
        case SHP_NODE_CONCAT:
            return shp_concat(&n.src[0], &n.src[1], n.op_params[0], y, st);
        case SHP_NODE_SUB:
            return shp_sub(&n.src[0], &n.src[1], y, st);
        case SHP_NODE_TANH:
            return shp_tanh(&n.src[0], y, st);
        case SHP_NODE_SIGMOID:
            return shp_sigmoid(&n.src[0], y, st);
        case SHP_NODE_ELU:
            return shp_elu(&n.src[0], y, st);
        case SHP_NODE_GELU_ERF:
            return shp_gelu_erf(&n.src[0], y, st);
        case SHP_NODE_CLAMP:
            return shp_clamp(&n.src[0], fparam(n, 0), fparam(n, 1), y, st);
        case SHP_NODE_NORM:
            return shp_norm(&n.src[0], fparam(n, 0), y, st);
        case SHP_NODE_IM2COL:
            return shp_im2col(&n.src[0], &n.src[1], n.op_params[0], n.op_params[2], n.op_params[4], y, st);
        case SHP_NODE_COL2IM_1D:
            return shp_col2im_1d(&n.src[0], n.op_params[0], n.op_params[1], n.op_params[2], y, st);
        case SHP_NODE_PAD: {
            const int32_t lp[4] = { n.op_params[0], n.op_params[2], n.op_params[4], n.op_params[6] };
            return shp_pad(&n.src[0], lp, y, st);
        }
        case SHP_NODE_PAD_REFLECT_1D:
            return shp_pad_reflect_1d(&n.src[0], n.op_params[0], n.op_params[1], y, st);
        case SHP_NODE_REPEAT:
            return shp_repeat(&n.src[0], y, st);
        case SHP_NODE_RELU:
            return shp_relu(&n.src[0], y, st);
        case SHP_NODE_NEG:
            return shp_neg(&n.src[0], y, st);
        case SHP_NODE_STEP:
            return shp_step(&n.src[0], y, st);
        case SHP_NODE_SQRT:
            return shp_sqrt(&n.src[0], y, st);
        case SHP_NODE_DIAG_MASK_INF:
            return shp_diag_mask_inf(&n.src[0], n.op_params[0], y, st);
        case SHP_NODE_SUM_ROWS:
            return shp_sum_rows(&n.src[0], y, st);
        case SHP_NODE_MEAN:
            return shp_mean(&n.src[0], y, st);
        case SHP_NODE_ACC:
            return shp_acc(&n.src[0], &n.src[1], n.op_params[0], n.op_params[1], n.op_params[2], n.op_params[3], y, st);
        default:
            return SHP_ERR_UNSUPPORTED;
    }
}

shp_status_t launch_run(const Planner & pl, const Launch & l, shp_stream_t st) {
    switch (l.kind) {
        case SHP_RUN_NOP:
            return SHP_OK;
        case SHP_RUN_SINGLE:
            return launch_single(pl.node(l.first), st);
        case SHP_RUN_NORM_MUL:
            return shp_rms_norm_mul(l.x, l.w, l.f0, l.y, st);
        case SHP_RUN_NORM_MUL_ROPE:
            return shp_qk_norm_rope(l.x, nullptr, l.w, nullptr, l.f0, l.b, l.i0, l.f1, l.f2, l.y, nullptr, st);
        case SHP_RUN_ADD_NORM_MUL:
            return shp_add_rms_norm_mul(l.x, l.b, l.w, l.f0, l.sum, l.y, st);
        case SHP_RUN_SILU_MUL:
            return shp_swiglu(l.x, l.b, l.y, st);
        case SHP_RUN_ADD_LEAKY:
            return shp_add_leaky_relu(l.x, l.b, l.f0, l.sum, l.y, st);
        case SHP_RUN_ADD_SCALE_LEAKY:
            return shp_sum_scale_leaky_relu(l.terms.data(), static_cast<int32_t>(l.terms.size()), l.f0, l.f1, l.sum,
                                            l.y, st);
        case SHP_RUN_SNAKE:
            return shp_snake(l.x, l.w, l.y, st);
        case SHP_RUN_SNAKE_GUARDED:
            return shp_snake_guarded(l.x, l.w, l.y, st);
        case SHP_RUN_SNAKE_BETA:
            return shp_snake_beta(l.x, l.w, l.c1, l.y, st);
        case SHP_RUN_GATHER_SUM:
            return shp_get_rows_sum(l.terms.data(), static_cast<int32_t>(l.terms.size()), &l.codes, l.y, st);
        case SHP_RUN_QK_NORM_ROPE:
            return shp_qk_norm_rope(l.x, l.x2, l.w, l.w2, l.f0, l.b, l.i0, l.f1, l.f2, l.y, l.y2, st);
        case SHP_RUN_QK_NORM_ROPE_KV:
            // the copies' destinations are the cache views themselves (filled 0)
            return shp_qk_norm_rope_kv(l.x, l.x2, l.x3, l.w, l.w2, l.f0, l.b, l.i0, l.f1, l.f2, l.y, l.y2, l.y3, 0, st);
        case SHP_RUN_CONT_ADD_LEAKY:
            return shp_cont_add_leaky_relu(l.own_x ? &l.xv : l.x, l.own_b ? &l.bv : l.b, l.x3, l.i0, l.f0, l.sum,
                                           l.y, st);
        case SHP_RUN_VIEW_BINARY:
            return l.i0 == SHP_NODE_ADD ? shp_add(l.x, l.b, l.y, st) :
                   l.i0 == SHP_NODE_MUL ? shp_mul(l.x, l.b, l.y, st) :
                                          shp_div(l.x, l.b, l.y, st);
        case SHP_RUN_MUL_SUM_ROWS:
            return shp_mul_sum_rows(l.x, l.b, l.y, st);
        case SHP_RUN_DIAG_MASK_SOFT_MAX:
            return shp_soft_max_causal(l.x, l.i0, l.f0, l.y, st);
        case SHP_RUN_CONT_IM2COL:
            return shp_im2col(l.w, &l.xv, l.i0, l.i1, l.i2, l.y, st);
        default:
            return SHP_ERR_UNSUPPORTED;
    }
}

}  // namespace
}  // namespace shp

extern "C" int32_t shp_graph_node_supported(const shp_node * node) {
    if (node == nullptr || node->uses < 0 || node->op < 0 || node->op >= SHP_NODE_OP_COUNT) {
        return 0;
    }
    return shp::single_ok(*node) ? 1 : 0;
}

extern "C" shp_status_t shp_graph_plan(const shp_node * nodes,
                                       int32_t          n_nodes,
                                       shp_graph_run *  runs,
                                       int32_t          capacity,
                                       int32_t *        n_runs) {
    if (n_runs == nullptr || n_nodes < 0 || (n_nodes > 0 && nodes == nullptr) || (runs != nullptr && capacity < 0)) {
        return SHP_ERR_INVALID_ARG;
    }
    shp::Planner       pl(nodes, n_nodes);
    const shp_status_t st = pl.init();
    if (st != SHP_OK) {
        return st;
    }
    const auto plan = pl.plan();
    *n_runs         = static_cast<int32_t>(plan.size());
    if (runs != nullptr) {
        if (static_cast<int64_t>(plan.size()) > capacity) {
            return SHP_ERR_INVALID_ARG;
        }
        for (size_t r = 0; r < plan.size(); ++r) {
            runs[r].kind  = plan[r].kind;
            runs[r].first = plan[r].first;
            runs[r].last  = plan[r].last;
            runs[r].nodes = plan[r].count;
        }
    }
    return SHP_OK;
}

extern "C" shp_status_t shp_graph_compute(const shp_node * nodes, int32_t n_nodes, shp_stream_t stream) {
    if (n_nodes < 0 || (n_nodes > 0 && nodes == nullptr)) {
        return SHP_ERR_INVALID_ARG;
    }
    shp::Planner pl(nodes, n_nodes);
    shp_status_t st = pl.init();
    if (st != SHP_OK) {
        return st;
    }
    const auto plan = pl.plan();
    for (const auto & l : plan) {
        if (l.kind == SHP_RUN_UNSUPPORTED) {
            return SHP_ERR_UNSUPPORTED;
        }
    }
    for (const auto & l : plan) {
        if ((st = shp::launch_run(pl, l, stream)) != SHP_OK) {
            return st;
        }
    }
    return SHP_OK;
}
