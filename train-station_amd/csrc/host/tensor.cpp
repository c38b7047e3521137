// Tensor construction, recorded forward ops and their backward formulas.
// Each op launches one or two kernels of ts_hip.h on the library stream; no
// op synchronises except data()/value().
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <tuple>
#include <sstream>

#include "ts_hip.h"
#include "ts_host.h"

namespace ts {

std::string dims_str(const std::vector<size_t> &d) {
    std::ostringstream os;
    os << "[";
    for (size_t i = 0; i < d.size(); ++i) os << (i ? ", " : "") << d[i];
    os << "]";
    return os.str();
}

namespace {

void *S() { return Runtime::get().stream(); }

// One 2-D product (with its optional epilogue) through ts_hip_gemm_fused; a
// split product's temporary comes from the pool, so no op allocates on the
// library stream (which keeps every step recordable as a HIP graph).
int gemm2d(int ta, int tb, size_t M, size_t N, size_t K, const float *A, size_t lda, const float *B, size_t ldb,
           const float *bias, bool relu, const float *mask, float *C, size_t ldc) {
    const size_t ws = ts_hip_gemm_workspace_floats(M, N, K);
    std::unique_ptr<Allocation> work;  // back to the pool on return: later work is stream-ordered after it
    if (ws) work = std::make_unique<Allocation>(ws);
    return ts_hip_gemm_fused(ta, tb, M, N, K, A, lda, B, ldb, bias, relu ? 1 : 0, mask, C, ldc,
                             work ? work->get() : nullptr, ws, S());
}

size_t product(const std::vector<size_t> &d) {
    size_t n = 1;
    for (size_t x : d) n *= x;
    return n;
}

// Reference AVX2 body/tail split: 8-wide for negate and Adam
// (core/utils.rs:856-865, adam/mod.rs:727-773), 32-wide unrolled body for the
// division zero check (ops/div.rs:356-417).
size_t tail8(size_t n) { return (n / 8) * 8; }
size_t tail32(size_t n) { return (n / 32) * 32; }

int opcode(GradFn::Kind k) {
    switch (k) {
        case GradFn::Kind::Add: return 0;
        case GradFn::Kind::Sub: return 1;
        case GradFn::Kind::Mul: return 2;
        default: return 3;
    }
}

// out = a op b (same shape)
Tensor same_shape(const float *a, const float *b, const std::vector<size_t> &dims, int op) {
    Tensor out = Tensor::new_uninit(dims);
    const size_t n = out.size();
    float *o = out.dev_mut();
    auto &rt = Runtime::get();
    launch(KernelClass::Elementwise, 12.0 * n, "elementwise", [&] {
        switch (op) {
            case 0: return ts_hip_add(a, b, o, n, S());
            case 1: return ts_hip_sub(a, b, o, n, S());
            case 2: return ts_hip_mul(a, b, o, n, S());
            default: return ts_hip_div(a, b, o, n, tail32(n), rt.zero_index(), S());
        }
    });
    return out;
}

// out[r][c] = m[r][c] op v[c]   (or v[c] op m[r][c] when vec_first)
Tensor row_bcast(const float *m, const float *v, size_t rows, size_t cols, int op, bool vec_first) {
    Tensor out = Tensor::new_uninit({rows, cols});
    const size_t n = rows * cols;
    launch(KernelClass::Elementwise, 8.0 * n + 4.0 * cols, "row broadcast", [&] {
        return ts_hip_row_broadcast(op, m, v, out.dev_mut(), rows, cols, vec_first, tail32(n),
                                    Runtime::get().zero_index(), S());
    });
    return out;
}

Tensor map_unary(uint8_t code, const Tensor &x, float imm);
bool defer_ok(size_t n);

Tensor neg_of(const Tensor &x) {
    if (defer_ok(x.size())) return map_unary(TS_HIP_MAP_NEG, x, 0.0f);
    Tensor out = Tensor::new_uninit(x.dims());
    const size_t n = x.size();
    launch(KernelClass::Elementwise, 8.0 * n, "ts_hip_neg",
           [&] { return ts_hip_neg(x.dev(), out.dev_mut(), n, tail8(n), S()); });
    return out;
}

// compute_broadcast_shape (ops/broadcasting.rs:320-357): NumPy rules, axes
// aligned to the right; panics with the reference's message otherwise.
std::vector<size_t> broadcast_dims(const std::vector<size_t> &a, const std::vector<size_t> &b) {
    const size_t ra = a.size(), rb = b.size(), r = ra > rb ? ra : rb;
    std::vector<size_t> out(r);
    for (size_t i = 0; i < r; ++i) {
        const size_t da = i < ra ? a[ra - 1 - i] : 1, db = i < rb ? b[rb - 1 - i] : 1;
        if (da == db || db == 1) out[r - 1 - i] = da;
        else if (da == 1) out[r - 1 - i] = db;
        else
            throw Error("Cannot broadcast tensor shapes " + dims_str(a) + " and " + dims_str(b) +
                        ": Cannot broadcast shapes " + dims_str(a) + " and " + dims_str(b) +
                        ": incompatible dimensions at axis " + std::to_string(r - 1 - i));
    }
    if (r > TS_HIP_MAX_RANK) throw Error("broadcasting supports tensors of rank up to 8");
    return out;
}

// The broadcast operand materialised on the device (create_broadcast_tensor,
// broadcasting.rs:409-433), optionally scaled.
Tensor bcast_to(const float *src, const std::vector<size_t> &src_dims, const std::vector<size_t> &dims,
                float scale = 1.0f, bool use_scale = false) {
    Tensor out = Tensor::new_uninit(dims);
    if (out.size())
        launch(KernelClass::Elementwise, 8.0 * out.size(), "ts_hip_broadcast_copy", [&] {
            return ts_hip_broadcast_copy(src, src_dims.data(), src_dims.size(), out.dev_mut(), dims.data(),
                                         dims.size(), scale, use_scale ? 1 : 0, S());
        });
    return out;
}

// Sum of x over the axes in `mask` into a tensor of `out_dims` (the keepdim
// layout, possibly with the size-1 axes removed: the same element order).
Tensor reduce_axes(const float *x, const std::vector<size_t> &dims, unsigned mask, std::vector<size_t> out_dims,
                   float scale = 1.0f, bool use_scale = false) {
    if (dims.size() > TS_HIP_MAX_RANK) throw Error("reductions support tensors of rank up to 8");
    Tensor out = Tensor::new_uninit(std::move(out_dims));
    const size_t n_in = product(dims);
    if (out.size())
        launch(KernelClass::Reduction, 4.0 * n_in + 4.0 * out.size(), "ts_hip_reduce_sum", [&] {
            return ts_hip_reduce_sum(x, dims.data(), dims.size(), mask, out.dev_mut(), scale, use_scale ? 1 : 0,
                                     S());
        });
    return out;
}

void add_reader(const std::shared_ptr<Allocation> &input, const std::shared_ptr<Allocation> &reader);

// reduce_gradient_to_shape (grad_fn/utils.rs:23-60): sum over the leading axes
// broadcasting added and over the axes broadcast from size 1, as one
// reduction (the reference chains sum_dims calls; the sums agree to
// rounding).  [B, N] -> [N] uses the column-sum kernel.
Tensor reduce_to(const Tensor &g, const std::vector<size_t> &target) {
    if (g.dims() == target) return g.alias();
    const std::vector<size_t> &gd = g.dims();
    if (gd.size() == 2 && target.size() == 1 && target[0] == gd[1]) {
        const size_t rows = gd[0], cols = gd[1];
        Tensor out = Tensor::new_uninit({cols});
        if (fusion_enabled() && rows && cols && g.allocation()) {  // deferred: a bias gradient, see PendingColsum
            auto p = std::make_shared<PendingColsum>();
            p->src = g.allocation();
            p->rows = rows;
            p->cols = cols;
            add_reader(p->src, out.allocation());
            out.allocation()->colsum = std::move(p);
            return out;
        }
        const size_t ws = ts_hip_sum_dim0_workspace_floats(rows, cols);
        Allocation work(ws);
        launch(KernelClass::Reduction, 4.0 * rows * cols + 4.0 * cols, "ts_hip_sum_dim0", [&] {
            return ts_hip_sum_dim0(g.dev(), rows, cols, out.dev_mut(), work.get(), ws, S());
        });
        return out;
    }
    if (target.size() > gd.size()) throw Error("reduce_gradient_to_shape: target has more axes than the gradient");
    const size_t lead = gd.size() - target.size();
    unsigned mask = 0;
    for (size_t k = 0; k < gd.size(); ++k) {
        if (k < lead) mask |= 1u << k;
        else if (target[k - lead] == 1 && gd[k] > 1) mask |= 1u << k;
        else if (target[k - lead] != gd[k])
            throw Error("reduce_gradient_to_shape: " + dims_str(gd) + " -> " + dims_str(target));
    }
    return reduce_axes(g.dev(), gd, mask, target);
}

bool is_row_broadcast(const std::vector<size_t> &full, const std::vector<size_t> &v) {
    return full.size() == 2 && v.size() == 1 && v[0] == full[1];
}

// go (full shape) op broadcast(x): x itself when it has the full shape, the
// row-broadcast kernel for a [N] vector over [B, N], else x materialised.
Tensor with_bcast(const Tensor &go, const SavedTensor &x, int op) {
    if (x.dims == go.dims()) return same_shape(go.dev(), x.ptr(), go.dims(), op);
    if (is_row_broadcast(go.dims(), x.dims))
        return row_bcast(go.dev(), x.ptr(), go.dims()[0], go.dims()[1], op, false);
    Tensor xb = bcast_to(x.ptr(), x.dims, go.dims());
    return same_shape(go.dev(), xb.dev(), go.dims(), op);
}

// softmax's [outer, reduce, inner] view of an axis
void axis_view(const std::vector<size_t> &dims, size_t dim, size_t &outer, size_t &reduce, size_t &inner) {
    outer = 1;
    inner = 1;
    for (size_t k = 0; k < dim; ++k) outer *= dims[k];
    reduce = dims[dim];
    for (size_t k = dim + 1; k < dims.size(); ++k) inner *= dims[k];
}

}  // namespace

// ---- deferred products ------------------------------------------------------

namespace {
bool g_fusion = true;

void add_reader(const std::shared_ptr<Allocation> &input, const std::shared_ptr<Allocation> &reader) {
    if (!input) return;
    auto &rs = input->readers;
    size_t live = 0;  // drop readers that are gone or already produced
    for (auto &w : rs) {
        auto r = w.lock();
        if (r && r->deferred()) rs[live++] = w;
    }
    rs.resize(live);
    rs.push_back(reader);
}
}  // namespace

void set_fusion(bool on) { g_fusion = on; }
bool fusion_enabled() { return g_fusion; }

void set_pending(const std::shared_ptr<Allocation> &out, std::shared_ptr<PendingGemm> p) {
    add_reader(p->A, out);
    add_reader(p->B, out);
    add_reader(p->src, out);
    add_reader(p->bias, out);
    add_reader(p->sub, out);
    add_reader(p->mask, out);
    out->pending = std::move(p);
}

void materialize_colsum(Allocation &a) {
    const std::shared_ptr<PendingColsum> p = std::move(a.colsum);
    a.colsum.reset();
    const float *x = p->src->get();
    const size_t rows = p->rows, cols = p->cols;
    const size_t ws = ts_hip_sum_dim0_workspace_floats(rows, cols);
    Allocation work(ws);
    launch(KernelClass::Reduction, 4.0 * rows * cols + 4.0 * cols, "ts_hip_sum_dim0", [&] {
        return ts_hip_sum_dim0(x, rows, cols, a.raw(), work.get(), ws, S());
    });
}

std::shared_ptr<PendingGemm> new_product(const std::shared_ptr<Allocation> &out) {
    auto p = std::make_shared<PendingGemm>();
    p->group = std::make_shared<ProductGroup>();
    p->group->bare = out;
    p->group->members.push_back(out);
    return p;
}

std::shared_ptr<PendingGemm> fork_pending(const std::shared_ptr<Allocation> &src, const std::shared_ptr<Allocation> &out) {
    if (!src || !src->pending) return nullptr;
    auto p = std::make_shared<PendingGemm>(*src->pending);
    if (p->group) p->group->members.push_back(out);
    return p;
}

namespace {

// The group's other members whose records still run its product.
std::vector<std::shared_ptr<Allocation>> pending_members(const Allocation &a, const PendingGemm &p) {
    std::vector<std::shared_ptr<Allocation>> out;
    if (!p.group) return out;
    auto &ms = p.group->members;
    size_t live = 0;
    for (auto &w : ms) {
        auto m = w.lock();
        if (!m || !m->pending || m->pending->src || m->pending->group != p.group) continue;
        ms[live++] = w;
        if (m.get() != &a) out.push_back(std::move(m));
    }
    ms.resize(live);
    return out;
}

// A deferred elementwise value that is a single chain of ops over one
// per-element buffer, each op's other operand a constant (relu's backward of
// the seed, the MSE's gradient 2 * d * (1/n)): that buffer, and the chain as
// a GEMM operand transform (ts_hip_operand_xf), so a product reads the buffer
// and the value itself is never stored.  False for anything else, or a chain
// that does not keep +0 (the transform's condition).  The ops map one to
// one: x op c is the _S op, c - x and c / x the reversed ones, c * x and
// c + x the _S op (c not a NaN, so the operands' order cannot show); a
// division checked for zero divisors, relu's backward with a constant
// input and negation (whose sign rule depends on the index) do not map.
bool operand_xf(const std::shared_ptr<Allocation> &al, std::shared_ptr<Allocation> &leaf, ts_hip_operand_xf &xf) {
    if (!fusion_enabled() || !al || !al->map) return false;
    const PendingMap &m = *al->map;
    int vl = -1;  // the per-element buffer
    for (size_t k = 0; k < m.leaves.size(); ++k) {
        if ((m.consts >> k) & 1u) continue;
        if (((m.scalar >> k) & 1u) || vl >= 0) return false;
        vl = static_cast<int>(k);
    }
    if (vl < 0 || m.root < 0) return false;
    auto const_of = [&](int j, float &c) {
        const MapNode &nd = m.nodes[j];
        if (nd.code != MapNode::kLeaf || !((m.consts >> nd.a) & 1u)) return false;
        c = m.values[nd.a];
        return true;
    };
    auto chain_op = [&](int j, uint8_t &code, float &c, int &next) {
        const MapNode &nd = m.nodes[j];
        next = nd.a;
        c = nd.imm;
        switch (nd.code) {
            case TS_HIP_MAP_ADD_S: code = TS_HIP_XF_ADD_S; return true;
            case TS_HIP_MAP_SUB_S: code = TS_HIP_XF_SUB_S; return true;
            case TS_HIP_MAP_MUL_S: code = TS_HIP_XF_MUL_S; return true;
            case TS_HIP_MAP_DIV_S: code = TS_HIP_XF_DIV_S; return true;
            case TS_HIP_MAP_RELU: code = TS_HIP_XF_RELU; return true;
            case TS_HIP_MAP_SQUARE: code = TS_HIP_XF_SQUARE; return true;
            case TS_HIP_MAP_ADD:
            case TS_HIP_MAP_MUL:
                code = nd.code == TS_HIP_MAP_ADD ? TS_HIP_XF_ADD_S : TS_HIP_XF_MUL_S;
                if (const_of(nd.b, c)) return true;
                next = nd.b;
                return const_of(nd.a, c) && !std::isnan(c);
            case TS_HIP_MAP_SUB:
                code = TS_HIP_XF_SUB_S;
                if (const_of(nd.b, c)) return true;
                code = TS_HIP_XF_RSUB_S;
                next = nd.b;
                return const_of(nd.a, c);
            case TS_HIP_MAP_DIV:
                if (nd.flags & TS_HIP_MAP_CHECKED) return false;
                code = TS_HIP_XF_DIV_S;
                if (const_of(nd.b, c)) return true;
                code = TS_HIP_XF_RDIV_S;
                next = nd.b;
                return const_of(nd.a, c);
            case TS_HIP_MAP_RELU_BWD:
                code = TS_HIP_XF_RELU_BWD_S;
                return const_of(nd.b, c);
            default:
                return false;
        }
    };
    uint8_t codes[TS_HIP_XF_MAX_OPS];
    float imms[TS_HIP_XF_MAX_OPS];
    int len = 0;
    for (int j = m.root; !(m.nodes[j].code == MapNode::kLeaf && m.nodes[j].a == vl);) {
        if (m.nodes[j].code == MapNode::kLeaf || len == TS_HIP_XF_MAX_OPS) return false;
        int next;
        if (!chain_op(j, codes[len], imms[len], next)) return false;
        ++len;
        j = next;
    }
    int ops = 0;  // nothing else computed in the program
    for (const MapNode &nd : m.nodes) ops += nd.code != MapNode::kLeaf;
    if (ops != len || len == 0) return false;
    xf = ts_hip_operand_xf{};
    xf.n_ops = static_cast<uint32_t>(len);
    float z = 0.0f;  // +0 through the chain, innermost op first
    for (int i = 0; i < len; ++i) {
        xf.code[i] = codes[len - 1 - i];
        xf.imm[i] = imms[len - 1 - i];
        const float c = xf.imm[i];
        switch (xf.code[i]) {
            case TS_HIP_XF_ADD_S: z = z + c; break;
            case TS_HIP_XF_SUB_S: z = z - c; break;
            case TS_HIP_XF_MUL_S: z = z * c; break;
            case TS_HIP_XF_DIV_S: z = z / c; break;
            case TS_HIP_XF_RSUB_S: z = c - z; break;
            case TS_HIP_XF_RDIV_S: z = c / z; break;
            case TS_HIP_XF_RELU: z = z > 0.0f ? z : 0.0f; break;
            case TS_HIP_XF_RELU_BWD_S: z = z > 0.0f ? c : 0.0f; break;
            default: z = z * z; break;
        }
    }
    uint32_t bits;
    std::memcpy(&bits, &z, 4);
    if (bits != 0) return false;
    leaf = m.leaves[vl];
    return true;
}

// gemm2d with operand transforms (null: none)
int gemm2d_xf(int ta, int tb, size_t M, size_t N, size_t K, const float *A, size_t lda, const ts_hip_operand_xf *xa,
              const float *B, size_t ldb, const ts_hip_operand_xf *xb, const float *bias, bool relu,
              const float *mask, float *C, size_t ldc) {
    const size_t ws = ts_hip_gemm_workspace_floats(M, N, K);
    std::unique_ptr<Allocation> work;
    if (ws) work = std::make_unique<Allocation>(ws);
    return ts_hip_gemm_fused_xf(ta, tb, M, N, K, A, lda, xa, B, ldb, xb, bias, relu ? 1 : 0, mask, C, ldc,
                                work ? work->get() : nullptr, ws, S());
}

std::vector<std::weak_ptr<Allocation>> &pending_reduces();

// A deferred sum / mean still to be formed of all n values of x, or of a
// chain of ops over x alone that a transform expresses (xs: that chain, or
// no ops), or null.
std::shared_ptr<Allocation> pending_sum_of(const std::shared_ptr<Allocation> &x, size_t n, ts_hip_operand_xf &xs) {
    for (auto &w : pending_reduces()) {
        auto o = w.lock();
        if (!o || !o->reduce || o->reduce->n != n) continue;
        xs = ts_hip_operand_xf{};
        if (o->reduce->x == x) return o;
        std::shared_ptr<Allocation> leaf;
        if (operand_xf(o->reduce->x, leaf, xs) && leaf == x) return o;
    }
    xs = ts_hip_operand_xf{};
    return nullptr;
}

// A product's operands as its launch reads them: fetched (deferred inputs
// run now), an operand that is a deferred chain over one buffer read as that
// buffer with the chain applied as it is loaded.
struct ProductOperands {
    const float *A = nullptr, *B = nullptr, *bias = nullptr, *sub = nullptr, *mask = nullptr;
    ts_hip_operand_xf xa{}, xb{};
    bool fa = false, fb = false;
};

ProductOperands product_operands(const PendingGemm &p, bool with_epilogue) {
    ProductOperands o;
    if (with_epilogue && p.sub) {  // the narrow kernel's subtraction (no operand transforms)
        o.A = p.A->get();
        o.B = p.B->get();
        o.bias = p.bias ? p.bias->get() : nullptr;
        o.sub = p.sub->get();
        o.mask = p.mask ? p.mask->get() : nullptr;
        return o;
    }
    std::shared_ptr<Allocation> la, lb;
    const bool takes = ts_hip_gemm_takes_xf(p.ta, p.tb, p.M, p.N, p.K, 0) != 0;
    o.fa = takes && operand_xf(p.A, la, o.xa);
    o.fb = takes && operand_xf(p.B, lb, o.xb);
    o.A = o.fa ? la->get() : p.A->get();
    o.B = o.fb ? lb->get() : p.B->get();
    o.bias = with_epilogue && p.bias ? p.bias->get() : nullptr;
    o.mask = with_epilogue && p.mask ? p.mask->get() : nullptr;
    return o;
}

void issue_product(const PendingGemm &p, const ProductOperands &o, float *C, bool with_epilogue) {
    DevicePool::get().note_use(C);  // a step being recorded writes it on every replay
    if (with_epilogue && p.sub) {
        launch(KernelClass::Gemm, 2.0 * p.M * p.N * p.K, "ts_hip_gemm_fused_sub", [&] {
            return ts_hip_gemm_fused_sub(p.ta, p.tb, p.M, p.N, p.K, o.A, p.lda, o.B, p.ldb, o.bias, o.sub,
                                         p.relu ? 1 : 0, o.mask, C, p.N, S());
        });
        return;
    }
    const bool relu = with_epilogue && p.relu;
    launch(KernelClass::Gemm, 2.0 * p.M * p.N * p.K, "ts_hip_gemm_fused", [&] {
        if (o.fa || o.fb)
            return gemm2d_xf(p.ta, p.tb, p.M, p.N, p.K, o.A, p.lda, o.fa ? &o.xa : nullptr, o.B, p.ldb,
                             o.fb ? &o.xb : nullptr, o.bias, relu, o.mask, C, p.N);
        return gemm2d(p.ta, p.tb, p.M, p.N, p.K, o.A, p.lda, o.B, p.ldb, o.bias, relu, o.mask, C, p.N);
    });
}

// inputs first (they may be deferred themselves), outside this launch's window
void launch_product(const PendingGemm &p, float *C, bool with_epilogue) {
    const ProductOperands o = product_operands(p, with_epilogue);
    issue_product(p, o, C, with_epilogue);
}

void finish_sibling(SiblingLaunch &s) {
    s.done = true;
    for (auto &w : s.outputs)
        if (auto o = w.lock())
            if (o->sibling.get() == &s) o->sibling.reset();
}

// The product of p, with the weight-gradient product held beside it (if any,
// and unless a group is already forming on this thread) in one launch group:
// the two run as one launch, timed as one.
void launch_product_grouped(const PendingGemm &p, float *C, bool with_epilogue) {
    const std::shared_ptr<SiblingLaunch> sib = p.sibling;
    LaunchCollector *&cur = launch_collector();
    if (!sib || sib->done || cur) {
        launch_product(p, C, with_epilogue);
        return;
    }
    // every input of both first (deferred ones run here, outside the group)
    const ProductOperands o = product_operands(p, with_epilogue);
    for (auto &in : sib->inputs)
        if (in) in->get();
    Profiler &P = Profiler::get();
    LaunchCollector col;
    P.begin(KernelClass::Gemm);
    const int st = ts_hip_launch_group_begin(S());
    if (st != TS_HIP_OK) {
        P.abort();
        check(st, "ts_hip_launch_group_begin");
    }
    cur = &col;
    try {
        issue_product(p, o, C, with_epilogue);
        sib->run();
    } catch (...) {
        cur = nullptr;
        (void)ts_hip_launch_group_end(S());  // what was held is launched
        P.abort();
        throw;
    }
    cur = nullptr;
    const int end = ts_hip_launch_group_end(S());
    if (end != TS_HIP_OK) {
        P.abort();
        check(end, "ts_hip_launch_group_end");
    }
    P.end(KernelClass::Gemm, col.work);
    finish_sibling(*sib);
}

}  // namespace

LaunchCollector *&launch_collector() {
    static thread_local LaunchCollector *c = nullptr;
    return c;
}

void run_sibling(Allocation &a) {
    // the record stays until the launch has succeeded (as for a product)
    const std::shared_ptr<SiblingLaunch> s = a.sibling;
    if (!s->done) s->run();
    finish_sibling(*s);
}

void materialize(Allocation &a) {
    // The record stays until the launch has succeeded: after a failed launch
    // the next read of the buffer tries again (and reports the error again)
    // instead of returning contents that were never written.
    const std::shared_ptr<PendingGemm> p = a.pending;
    float *C = a.raw();
    if (p->src) {  // epilogue only: the separate kernels, in the fused epilogue's order
        const float *x = p->src->get();
        const float *bias = p->bias ? p->bias->get() : nullptr;
        const float *sub = p->sub ? p->sub->get() : nullptr;
        const float *mask = p->mask ? p->mask->get() : nullptr;
        DevicePool::get().note_use(C);
        const size_t n = p->M * p->N;
        if (bias) {
            launch(KernelClass::Elementwise, 8.0 * n + 4.0 * p->N, "ts_hip_bias_add",
                   [&] { return ts_hip_bias_add(x, bias, C, p->M, p->N, 0, S()); });
            x = C;
        }
        if (sub) {
            launch(KernelClass::Elementwise, 12.0 * n, "ts_hip_sub", [&] { return ts_hip_sub(x, sub, C, n, S()); });
            x = C;
        }
        if (p->relu) {
            launch(KernelClass::Elementwise, 8.0 * n, "ts_hip_relu", [&] { return ts_hip_relu(x, C, n, S()); });
            x = C;
        }
        if (mask || x != C)
            launch(KernelClass::Elementwise, 12.0 * n, "ts_hip_relu_backward", [&] {
                return mask ? ts_hip_relu_backward(mask, x, C, n, S()) : ts_hip_copy(x, C, n, S());
            });
        a.pending.reset();
        return;
    }
    const std::vector<std::shared_ptr<Allocation>> others = pending_members(a, *p);
    if (others.empty()) {  // the only consumer: the product with its epilogue, in one launch
        launch_product_grouped(*p, C, true);
        a.pending.reset();
        return;
    }
    // Several consumers: the product once, bare, into its own buffer (or a
    // temporary when that was dropped); then every member keeps only its
    // epilogue, reading it.
    std::shared_ptr<Allocation> prod = p->group->bare.lock();
    if (!prod || !prod->pending || !prod->pending->bare() || prod->pending->group != p->group)
        prod = std::make_shared<Allocation>(p->M * p->N);
    launch_product_grouped(*p, prod->raw(), false);
    if (prod->pending) prod->pending.reset();
    std::vector<std::shared_ptr<Allocation>> all = others;
    all.push_back(a.shared_from_this());
    for (auto &m : all) {
        if (m == prod || !m->pending || m->pending->src) continue;
        const std::shared_ptr<PendingGemm> old = m->pending;
        auto e = std::make_shared<PendingGemm>();
        e->M = old->M;
        e->N = old->N;
        e->src = prod;
        e->bias = old->bias;
        e->sub = old->sub;
        e->relu = old->relu;
        e->mask = old->mask;
        set_pending(m, e);
    }
    if (a.pending) materialize(a);
}

// ---- deferred elementwise programs -------------------------------------------

namespace {

// The registers of a pass over program p: reg[j] for every node the pass
// computes, -1 for a node it need not (read by no computed op, not kept, no
// division to check).  Input k sits in register k from the start until its
// last use; each op then takes the lowest free register, after the registers
// of operands it reads for the last time are freed (an op reads its operands
// before it writes).  Nodes in `keep` -- the stored values and the summed one
// -- stay live to the end.  False when the computed ops exceed
// TS_HIP_MAP_MAX_OPS or more than TS_HIP_MAP_REGS values would be live at once.
bool allocate_registers(const PendingMap &p, const std::vector<int> &keep, std::vector<int> &reg) {
    const int n = static_cast<int>(p.nodes.size());
    constexpr int kEnd = 1 << 30;
    std::vector<int> last(n, -1);
    std::vector<char> need(n, 0);
    for (int j : keep) {
        need[j] = 1;
        last[j] = kEnd;
    }
    int ops = 0;
    for (int j = n - 1; j >= 0; --j) {
        const MapNode &nd = p.nodes[j];
        if (nd.code == MapNode::kLeaf || (!need[j] && nd.checks.empty())) continue;
        need[j] = 1;
        ++ops;
        for (const int o : {static_cast<int>(nd.a), static_cast<int>(nd.b)}) {
            need[o] = 1;
            if (last[o] < j) last[o] = j;
        }
    }
    if (ops > TS_HIP_MAP_MAX_OPS) return false;
    reg.assign(n, -1);
    uint32_t busy = 0;
    for (int j = 0; j < n; ++j) {
        const MapNode &nd = p.nodes[j];
        if (nd.code == MapNode::kLeaf && need[j]) {
            reg[j] = nd.a;
            busy |= 1u << nd.a;
        }
    }
    for (int j = 0; j < n; ++j) {
        const MapNode &nd = p.nodes[j];
        if (nd.code == MapNode::kLeaf || !need[j]) continue;
        if (last[nd.a] == j) busy &= ~(1u << reg[nd.a]);
        if (last[nd.b] == j) busy &= ~(1u << reg[nd.b]);
        int d = 0;
        while (d < TS_HIP_MAP_REGS && ((busy >> d) & 1u)) ++d;
        if (d == TS_HIP_MAP_REGS) return false;
        reg[j] = d;
        if (last[j] >= 0) busy |= 1u << d;  // a checked division nothing reads frees its register at once
    }
    return true;
}

// One program under construction: its leaves and nodes, common
// subexpressions shared (the same op on the same operands is one node).
struct MapBuilder {
    PendingMap p;
    std::map<std::tuple<uint8_t, uint8_t, int, int, uint32_t>, int> cse;

    int leaf_node(int k) {
        for (size_t j = 0; j < p.nodes.size(); ++j)
            if (p.nodes[j].code == MapNode::kLeaf && p.nodes[j].a == k) return static_cast<int>(j);
        MapNode nd;
        nd.a = static_cast<int16_t>(k);
        p.nodes.push_back(nd);
        return static_cast<int>(p.nodes.size()) - 1;
    }
    int leaf(const std::shared_ptr<Allocation> &al, bool scalar) {
        // a deferred constant is read as its value, whatever the element count
        if (al->map && al->map->constant()) return constant(*al->map->constant());
        for (size_t k = 0; k < p.leaves.size(); ++k)
            if (p.leaves[k] == al && (((p.scalar >> k) & 1u) != 0) == scalar) return leaf_node(static_cast<int>(k));
        const int k = static_cast<int>(p.leaves.size());
        p.leaves.push_back(al);
        p.values.push_back(0.0f);
        if (scalar) p.scalar |= 1u << k;
        return leaf_node(k);
    }
    // a constant: an input of the pass holding v for every element (one leaf
    // per distinct value, no buffer, nothing read per element)
    int constant(float v) {
        for (size_t k = 0; k < p.leaves.size(); ++k)
            if (((p.consts >> k) & 1u) && std::memcmp(&p.values[k], &v, 4) == 0) return leaf_node(static_cast<int>(k));
        const int k = static_cast<int>(p.leaves.size());
        p.leaves.push_back(nullptr);
        p.values.push_back(v);
        p.consts |= 1u << k;
        p.scalar |= 1u << k;
        return leaf_node(k);
    }
    bool is_const(int j, float v) const {
        const MapNode &nd = p.nodes[j];
        return nd.code == MapNode::kLeaf && ((p.consts >> nd.a) & 1u) && p.values[nd.a] == v;
    }
    // `inherit`: the checks of a checked division copied from another
    // program (none: a new division, which gets a check of its own)
    int op(uint8_t code, int a, int b, float imm = 0.0f, uint8_t flags = 0,
           const std::vector<std::shared_ptr<DivCheck>> *inherit = nullptr) {
        if (b < 0) b = a;
        // the constant one scaled by imm is imm exactly (the mean's gradient
        // of the seed)
        if (code == TS_HIP_MAP_MUL_S && a >= 0 && is_const(a, 1.0f)) return constant(imm);
        uint32_t bits;
        std::memcpy(&bits, &imm, 4);
        const auto key = std::make_tuple(code, flags, a, b, bits);
        auto it = cse.find(key);
        if (it != cse.end()) {
            if (inherit) {
                auto &mine = p.nodes[it->second].checks;
                for (const auto &c : *inherit)
                    if (std::find(mine.begin(), mine.end(), c) == mine.end()) mine.push_back(c);
            }
            return it->second;
        }
        MapNode nd;
        nd.code = code;
        nd.flags = flags;
        nd.a = static_cast<int16_t>(a);
        nd.b = static_cast<int16_t>(b);
        nd.imm = imm;
        if (inherit) nd.checks = *inherit;
        else if (flags & TS_HIP_MAP_CHECKED) nd.checks.push_back(std::make_shared<DivCheck>());
        p.nodes.push_back(std::move(nd));
        const int id = static_cast<int>(p.nodes.size()) - 1;
        cse.emplace(key, id);
        return id;
    }
    // m's program merged in; returns the node of its value, which records
    // `origin` (the allocation m was deferred for)
    int import(const PendingMap &m, const std::shared_ptr<Allocation> &origin) {
        std::vector<int> remap(m.nodes.size(), -1);
        for (size_t j = 0; j < m.nodes.size(); ++j) {
            const MapNode &nd = m.nodes[j];
            if (nd.code == MapNode::kLeaf) {
                remap[j] = ((m.consts >> nd.a) & 1u) ? constant(m.values[nd.a])
                                                     : leaf(m.leaves[nd.a], ((m.scalar >> nd.a) & 1u) != 0);
            } else {
                remap[j] = op(nd.code, remap[nd.a], remap[nd.b], nd.imm, nd.flags, &nd.checks);
                if (p.nodes[remap[j]].origin.expired() && !nd.origin.expired()) p.nodes[remap[j]].origin = nd.origin;
            }
        }
        const int r = remap[m.root];
        if (origin && p.nodes[r].code != MapNode::kLeaf) p.nodes[r].origin = origin;
        return r;
    }
    // the value of `al` (n elements): its deferred program merged in, or a leaf
    int value(const std::shared_ptr<Allocation> &al, size_t n) {
        if (al->map && al->map->n == n) return import(*al->map, al);
        return leaf(al, false);
    }
    // one pass can compute the program with the nodes of `keep` stored
    bool fits(const std::vector<int> &keep) const {
        std::vector<int> reg;
        return p.leaves.size() <= static_cast<size_t>(TS_HIP_MAP_MAX_INPUTS) && allocate_registers(p, keep, reg);
    }
};

// true when something besides `own` local references (and the division-check
// list) holds the allocation
bool held_elsewhere(const std::shared_ptr<Allocation> &a, long own) {
    return a.use_count() > own + (a->check_hold ? 1 : 0);
}

bool open_checks(const PendingMap &m) {
    for (const MapNode &nd : m.nodes)
        for (const auto &c : nd.checks)
            if (!c->done) return true;
    return false;
}

// This thread's deferred values whose programs hold a checked division that
// no pass has computed yet (only sizes with a tail: the check is on the
// elements past 32 * floor(n / 32)).  Held here so they run, before the next
// synchronisation reads the zero-divisor word, even when nothing else reads
// them; being registered readers of their inputs, they also run before an
// input is overwritten in place.
std::vector<std::shared_ptr<Allocation>> &check_holds() {
    static thread_local std::vector<std::shared_ptr<Allocation>> v;
    return v;
}

void prune_check_holds() {
    auto &v = check_holds();
    size_t k = 0;
    for (size_t i = 0; i < v.size(); ++i) {
        if (v[i]->map && open_checks(*v[i]->map)) v[k++] = std::move(v[i]);
        else v[i]->check_hold = false;
    }
    v.resize(k);
}

constexpr size_t kMaxCheckHolds = 256;  // past this the held programs run (bounds what they keep alive)

void hold_for_check(const std::shared_ptr<Allocation> &al) {
    if (al->check_hold) return;
    if (check_holds().size() >= kMaxCheckHolds) run_division_checks();
    check_holds().push_back(al);
    al->check_hold = true;
}

struct MapOutput {
    std::shared_ptr<Allocation> alloc;
    int node;
};

// This thread's deferred sums and means (outputs whose `reduce` is pending),
// for passes to take up as their reduction.
std::vector<std::weak_ptr<Allocation>> &pending_reduces() {
    static thread_local std::vector<std::weak_ptr<Allocation>> v;
    return v;
}

// A pass with no reduction of its own takes up a deferred sum of a value it
// can compute from the inputs it reads anyway (its program merged in, within
// the pass's limits): the sum costs the pass no extra reads.  `keep` gains the
// summed node.
void attach_reduce(MapBuilder &b, std::vector<int> &keep, int &reduce, float *&sum_out, bool &mean) {
    auto &v = pending_reduces();
    size_t live = 0;
    for (size_t i = 0; i < v.size(); ++i) {
        auto o = v[i].lock();
        if (!o || !o->reduce) continue;  // gone or computed: off the list
        const PendingReduce &r = *o->reduce;
        if (reduce < 0 && r.x->map && r.x->map->n == b.p.n) {
            MapBuilder trial = b;
            const int node = trial.import(*r.x->map, r.x);
            bool reads_more = trial.p.leaves.size() > static_cast<size_t>(TS_HIP_MAP_MAX_INPUTS);
            for (size_t q = b.p.leaves.size(); q < trial.p.leaves.size(); ++q)
                reads_more = reads_more || !((trial.p.consts >> q) & 1u);
            keep.push_back(node);
            std::vector<int> reg;
            if (!reads_more && allocate_registers(trial.p, keep, reg)) {
                b = std::move(trial);
                reduce = node;
                sum_out = o->raw();
                mean = r.mean;
                DevicePool::get().note_use(sum_out);
                o->reduce.reset();
                continue;
            }
            keep.pop_back();
        }
        v[live++] = v[i];
    }
    v.resize(live);
}

// Runs one program: stores `outs` (and, outside backward, any still-deferred
// origin the program computes on the way that something else holds, as far
// as the registers allow), and with sum_out set adds node `reduce` up as
// ts_hip_sum / ts_hip_mean would.
void launch_program(MapBuilder &b, std::vector<MapOutput> outs, int reduce = -1, float *sum_out = nullptr,
                    bool mean = false) {
    const size_t n = b.p.n;
    std::vector<int> keep, reg;
    for (const MapOutput &m : outs) keep.push_back(m.node);
    if (reduce >= 0) keep.push_back(reduce);
    else attach_reduce(b, keep, reduce, sum_out, mean);
    if (!allocate_registers(b.p, keep, reg)) throw Error("an elementwise program exceeds the fused pass's limits");
    // A value still held (a saved operand, or its tensor) may be read again,
    // and this pass computes it anyway, so it stores it -- except during
    // backward, whose passes run after the forward values' last graph use:
    // there a value read later is computed again from its inputs.
    for (size_t j = 0; !in_backward() && j < b.p.nodes.size() && outs.size() < static_cast<size_t>(TS_HIP_MAP_MAX_OUTPUTS);
         ++j) {
        auto o = b.p.nodes[j].origin.lock();
        if (!o || !o->map || !held_elsewhere(o, 1)) continue;
        bool listed = false;
        for (const MapOutput &m : outs) listed = listed || m.alloc == o;
        if (listed) continue;
        keep.push_back(static_cast<int>(j));
        std::vector<int> trial;
        if (allocate_registers(b.p, keep, trial)) {
            outs.push_back({o, static_cast<int>(j)});
            reg = std::move(trial);
        } else {
            keep.pop_back();
        }
    }
    // leaves first: deferred ones run before, outside this launch's window
    ts_hip_map_program prog{};
    prog.n_inputs = static_cast<uint32_t>(b.p.leaves.size());
    prog.scalar_inputs = b.p.scalar;
    prog.const_inputs = b.p.consts;
    double bytes = 0.0;
    std::vector<char> read(b.p.leaves.size(), 0);  // inputs a computed op or an output reads
    for (size_t j = 0; j < b.p.nodes.size(); ++j)
        if (b.p.nodes[j].code == MapNode::kLeaf && reg[j] >= 0) read[b.p.nodes[j].a] = 1;
    for (size_t k = 0; k < b.p.leaves.size(); ++k) {
        if (((b.p.consts >> k) & 1u) || !read[k]) {  // a constant (or an input nothing reads): no buffer
            prog.const_inputs |= 1u << k;
            prog.scalar_inputs |= 1u << k;
            prog.const_values[k] = read[k] ? b.p.values[k] : 0.0f;
            continue;
        }
        prog.inputs[k] = b.p.leaves[k]->get();
        if (!((b.p.scalar >> k) & 1u)) bytes += 4.0 * n;
    }
    for (size_t j = 0; j < b.p.nodes.size(); ++j) {
        const MapNode &nd = b.p.nodes[j];
        if (nd.code == MapNode::kLeaf || reg[j] < 0) continue;  // an input, or a value nothing needs
        ts_hip_map_op &op = prog.ops[prog.n_ops];
        op.code = nd.code;
        op.a = static_cast<uint8_t>(reg[nd.a]);
        op.b = static_cast<uint8_t>(reg[nd.b]);
        op.flags = nd.flags;
        op.imm = nd.imm;
        op.d = static_cast<uint8_t>(reg[j]);
        ++prog.n_ops;
    }
    for (const MapOutput &m : outs) {
        float *C = m.alloc->raw();
        DevicePool::get().note_use(C);  // a step being recorded writes it on every replay
        prog.outputs[prog.n_outputs] = C;
        prog.output_regs[prog.n_outputs] = static_cast<uint8_t>(reg[m.node]);
        ++prog.n_outputs;
        bytes += 4.0 * n;
    }
    prog.reduce_reg = reduce >= 0 ? reg[reduce] : -1;
    std::unique_ptr<Allocation> work;
    size_t wsf = 0;
    if (sum_out) {
        wsf = ts_hip_map_workspace_floats(n);
        work = std::make_unique<Allocation>(wsf);
    }
    Runtime &rt = Runtime::get();
    launch(KernelClass::Elementwise, bytes, "ts_hip_map", [&] {
        return ts_hip_map(&prog, n, tail8(n), tail32(n), rt.zero_index(), sum_out, mean ? 1 : 0,
                          work ? work->get() : nullptr, wsf, S());
    });
    for (const MapOutput &m : outs) m.alloc->map.reset();
    bool checked = false;
    for (const MapNode &nd : b.p.nodes)
        for (const auto &c : nd.checks) c->done = checked = true;
    if (checked) prune_check_holds();
}

// The deferred value of `dims` computed by build(builder, operand nodes) from
// `operands` (allocation, one-value-for-every-element); the operands' own
// deferred programs are merged in, or, if the result would exceed the program
// limits, run first and read as leaves.
template <class F>
std::shared_ptr<PendingMap> defer(size_t n, const std::vector<std::pair<std::shared_ptr<Allocation>, bool>> &operands,
                                  F &&build) {
    for (int attempt = 0; attempt < 2; ++attempt) {
        MapBuilder b;
        b.p.n = n;
        std::vector<int> ids;
        for (const auto &o : operands) ids.push_back(o.second ? b.leaf(o.first, true) : b.value(o.first, n));
        b.p.root = build(b, ids);
        if (b.fits({b.p.root})) return std::make_shared<PendingMap>(std::move(b.p));
        for (const auto &o : operands) o.first->get();
    }
    throw Error("an elementwise program exceeds the fused pass's limits");
}

// A new tensor of `dims` holding the deferred value p.
Tensor deferred_tensor(const std::vector<size_t> &dims, std::shared_ptr<PendingMap> p) {
    Tensor out = Tensor::new_uninit(dims);
    const auto &al = out.allocation();
    for (const auto &l : p->leaves) add_reader(l, al);
    al->map = std::move(p);
    if (tail32(al->map->n) < al->map->n && open_checks(*al->map)) hold_for_check(al);
    return out;
}

// Deferral applies to same-shape operands of at least one element with
// fusion on.
bool defer_ok(size_t n) { return fusion_enabled() && n > 0; }

Tensor map_binary(uint8_t code, const Tensor &x, const Tensor &y, uint8_t flags = 0) {
    auto p = defer(x.size(), {{x.allocation(), false}, {y.allocation(), false}},
                   [&](MapBuilder &b, const std::vector<int> &v) { return b.op(code, v[0], v[1], 0.0f, flags); });
    return deferred_tensor(x.dims(), std::move(p));
}

Tensor map_unary(uint8_t code, const Tensor &x, float imm = 0.0f) {
    auto p = defer(x.size(), {{x.allocation(), false}},
                   [&](MapBuilder &b, const std::vector<int> &v) { return b.op(code, v[0], -1, imm); });
    return deferred_tensor(x.dims(), std::move(p));
}

}  // namespace

void materialize_map(Allocation &a) { materialize_maps({a.shared_from_this()}); }

void run_division_checks() {
    std::vector<std::shared_ptr<Allocation>> open;
    for (const auto &a : check_holds())
        if (a->map && open_checks(*a->map)) open.push_back(a);
    if (!open.empty()) materialize_maps(open);
    prune_check_holds();
}

Tensor add_gradients(const Tensor &existing, const Tensor &g) {
    if (defer_ok(existing.size()) && existing.size() == g.size()) return map_binary(TS_HIP_MAP_ADD, existing, g);
    return same_shape(existing.dev(), g.dev(), existing.dims(), 0);
}

void materialize_maps(const std::vector<std::shared_ptr<Allocation>> &allocs) {
    MapBuilder group;
    std::vector<MapOutput> outs;
    auto flush = [&]() {
        if (!outs.empty()) launch_program(group, outs);
        group = MapBuilder();
        outs.clear();
    };
    for (const auto &al : allocs) {
        if (!al || !al->map) continue;
        bool listed = false;
        for (const MapOutput &m : outs) listed = listed || m.alloc == al;
        if (listed) continue;
        if (!outs.empty() && group.p.n == al->map->n && outs.size() < static_cast<size_t>(TS_HIP_MAP_MAX_OUTPUTS)) {
            MapBuilder trial = group;
            const int r = trial.import(*al->map, al);
            std::vector<int> keep{r};
            for (const MapOutput &m : outs) keep.push_back(m.node);
            if (trial.fits(keep)) {
                group = std::move(trial);
                outs.push_back({al, r});
                continue;
            }
        }
        flush();
        group.p.n = al->map->n;
        const int r = group.import(*al->map, al);
        outs.push_back({al, r});
    }
    flush();
}

size_t next_tensor_id() {
    // tensor/core/mod.rs:131: one process-wide atomic counter
    static std::atomic<size_t> counter{1};
    return counter.fetch_add(1, std::memory_order_relaxed);
}

// ---- construction ---------------------------------------------------------------

Tensor Tensor::new_uninit(std::vector<size_t> dims) {
    Tensor t;
    t.size_ = product(dims);
    t.dims_ = std::move(dims);
    t.id_ = next_tensor_id();
    if (t.size_ > 0) t.alloc_ = std::make_shared<Allocation>(t.size_);
    return t;
}

Tensor Tensor::filled(std::vector<size_t> dims, float v) {
    Tensor t = new_uninit(std::move(dims));
    if (t.size_)
        launch(KernelClass::Elementwise, 4.0 * t.size_, "ts_hip_fill",
               [&] { return ts_hip_fill(t.dev_mut(), v, t.size_, S()); });
    return t;
}

Tensor Tensor::constant(std::vector<size_t> dims, float v) {
    const size_t n = product(dims);
    if (!defer_ok(n)) return filled(std::move(dims), v);
    MapBuilder b;
    b.p.n = n;
    b.p.root = b.constant(v);
    return deferred_tensor(dims, std::make_shared<PendingMap>(std::move(b.p)));
}

Tensor Tensor::zeros(std::vector<size_t> dims) { return filled(std::move(dims), 0.0f); }
Tensor Tensor::ones(std::vector<size_t> dims) { return filled(std::move(dims), 1.0f); }

// XorShiftRng::new_from_time (random.rs:492-497) hashes the system time; any
// well-mixed 64-bit value of the clock serves (a splitmix64 finaliser of the
// nanosecond count plus a per-process counter, so two calls in the same tick
// still differ).
static uint64_t seed_from_time() {
    static std::atomic<uint64_t> calls{0};
    uint64_t z = static_cast<uint64_t>(std::chrono::system_clock::now().time_since_epoch().count()) +
                 0x9E3779B97F4A7C15ULL * (calls.fetch_add(1, std::memory_order_relaxed) + 1);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

void Tensor::fill_randn(const uint64_t *seed) {
    if (!size_) return;  // random.rs:271-273
    const uint64_t s = seed ? *seed : seed_from_time();
    alloc_->before_write();
    launch(KernelClass::Elementwise, 4.0 * size_, "ts_hip_randn",
           [&] { return ts_hip_randn(dev_mut(), size_, s, S()); });
}

Tensor Tensor::randn(std::vector<size_t> dims, const uint64_t *seed) {
    Tensor t = new_uninit(std::move(dims));
    t.fill_randn(seed);
    return t;
}

Tensor Tensor::from_slice(const float *data, size_t len, std::vector<size_t> dims) {
    const size_t n = product(dims);
    if (len != n)  // init/data.rs:227-247 returns Err on a length mismatch
        throw Error("Data length " + std::to_string(len) + " doesn't match shape " +
                    dims_str(dims) + " (size " + std::to_string(n) + ")");
    refuse_while_recording("from_slice");
    Tensor t = new_uninit(std::move(dims));
    if (n) {
        check(ts_hip_memcpy_async(t.dev_mut(), data, n, 0, S()), "ts_hip_memcpy_async");
        check(ts_hip_stream_synchronize(S()), "ts_hip_stream_synchronize");
    }
    return t;
}

Tensor Tensor::clone() const {
    Tensor t = new_uninit(dims_);
    if (size_)
        launch(KernelClass::Elementwise, 8.0 * size_, "ts_hip_copy",
               [&] { return ts_hip_copy(dev(), t.dev_mut(), size_, S()); });
    return t;
}

Tensor Tensor::alias() const {
    Tensor t;
    t.alloc_ = alloc_;
    t.dims_ = dims_;
    t.size_ = size_;
    t.id_ = next_tensor_id();
    return t;
}

Tensor Tensor::view() const {
    Tensor t;
    t.alloc_ = alloc_;
    t.dims_ = dims_;
    t.size_ = size_;
    t.id_ = id_;
    t.requires_grad_ = requires_grad_;
    t.strided_ = strided_;
    return t;
}

// ---- transpose, contiguous, fill (transform/transpose.rs, contiguous.rs,
// init/basic.rs) ---------------------------------------------------------------------

void materialize_transpose(Allocation &a) {
    const std::shared_ptr<PendingTranspose> p = a.transpose;
    const float *src = p->src->get();
    float *C = a.raw();
    DevicePool::get().note_use(C);
    launch(KernelClass::Elementwise, 8.0 * a.n, "ts_hip_transpose", [&] {
        return ts_hip_transpose(src, p->dims.data(), p->dims.size(), p->d0, p->d1, C, S());
    });
    a.transpose.reset();
}

namespace {
// A deferred copy of src (dims) with axes d0 and d1 swapped (d0 == d1: a
// plain copy) for `out`; a view reads src as it is when read, a copy is a
// reader of src and so runs before src is written in place.
void defer_transpose(const std::shared_ptr<Allocation> &out, const std::shared_ptr<Allocation> &src,
                     const std::vector<size_t> &dims, size_t d0, size_t d1, bool view) {
    auto t = std::make_shared<PendingTranspose>();
    t->src = src;
    t->dims = dims;
    t->d0 = d0;
    t->d1 = d1;
    t->view = view;
    if (!view) add_reader(src, out);
    out->transpose = std::move(t);
}

bool same_axes(const PendingTranspose &t, size_t d0, size_t d1) {
    return (t.d0 == d0 && t.d1 == d1) || (t.d0 == d1 && t.d1 == d0);
}
}  // namespace

Tensor transposed_value(const Tensor &x, size_t d0, size_t d1, bool view) {
    std::vector<size_t> od = x.dims();
    std::swap(od[d0], od[d1]);
    Tensor out = Tensor::new_uninit(od);
    const auto &a = x.allocation();
    if (!a || !out.size()) return out;
    if (a->transpose && a->transpose->d0 != a->transpose->d1 && same_axes(*a->transpose, d0, d1) &&
        a->transpose->dims == od) {
        // transposed back: the source's values (a copy, as the reference's
        // transpose of a strided view is, transpose.rs:187-190)
        defer_transpose(out.allocation(), a->transpose->src, od, 0, 0, false);
    } else if (od.size() == 2 && a->pending && a->pending->bare()) {
        // C = op(A) . op(B) not yet run: C^T = op(B)^T . op(A)^T, written
        // transposed by the product itself
        const PendingGemm &p = *a->pending;
        auto q = new_product(out.allocation());
        q->ta = p.tb ? 0 : 1;
        q->tb = p.ta ? 0 : 1;
        q->M = p.N;
        q->N = p.M;
        q->K = p.K;
        q->lda = p.ldb;
        q->ldb = p.lda;
        q->A = p.B;
        q->B = p.A;
        set_pending(out.allocation(), std::move(q));
    } else {
        defer_transpose(out.allocation(), a, x.dims(), d0, d1, view);
    }
    return out;
}

Tensor Tensor::transpose(size_t dim0, size_t dim1) const {
    const size_t rank = dims_.size();
    if (dim0 >= rank)  // transpose.rs:157-168
        throw Error("dim0 " + std::to_string(dim0) + " out of bounds for tensor with rank " + std::to_string(rank));
    if (dim1 >= rank)
        throw Error("dim1 " + std::to_string(dim1) + " out of bounds for tensor with rank " + std::to_string(rank));
    if (dim0 == dim1) return clone();  // :171-173: a clone, which tracks no gradient
    // a view of a contiguous tensor, a copy of a strided one (:181-186)
    const bool view = !strided_;
    Tensor out = transposed_value(*this, dim0, dim1, view);
    out.strided_ = view;
    if (requires_grad_) {  // :189-202, whatever is_grad_enabled() says
        GradFn fn{GradFn::Kind::Transpose};
        fn.dim0 = dim0;
        fn.dim1 = dim1;
        fn.input_shape = dims_;
        record(out, {id_}, std::move(fn));
    }
    return out;
}

Tensor Tensor::t() const {
    if (dims_.size() < 2)  // transpose.rs:283-291
        throw Error("Matrix transpose requires at least 2 dimensions, got " + std::to_string(dims_.size()));
    return transpose(dims_.size() - 2, dims_.size() - 1);
}

bool Tensor::is_contiguous() const { return !strided_; }

Tensor Tensor::contiguous() const {
    Tensor out;
    if (strided_ && alloc_ && alloc_->transpose && alloc_->transpose->view) {
        // the view's values as they are now, copied when first read
        const PendingTranspose &v = *alloc_->transpose;
        out = new_uninit(dims_);
        defer_transpose(out.alloc_, v.src, v.dims, v.d0, v.d1, false);
    } else {
        out = clone();  // contiguous.rs:124-137 (or a view already copied)
    }
    if (requires_grad_) {  // :125-157, whatever is_grad_enabled() says
        GradFn fn{GradFn::Kind::Contiguous};
        fn.input_shape = dims_;
        record(out, {id_}, std::move(fn));
    }
    return out;
}

void Tensor::fill(float value) {
    if (!size_) return;  // basic.rs:305-307
    Allocation *target = alloc_.get();
    // a view not yet copied writes through to its source, as the reference's
    // strided view shares its storage (every element of the source is one of
    // the view's)
    while (target->transpose && target->transpose->view) target = target->transpose->src.get();
    target->before_write();
    float *p = target->get();
    launch(KernelClass::Elementwise, 4.0 * size_, "ts_hip_fill", [&] { return ts_hip_fill(p, value, size_, S()); });
}

Tensor Tensor::from_saved(const SavedTensor &s) {
    Tensor t;
    t.alloc_ = s.alloc;
    t.dims_ = s.dims;
    t.size_ = product(s.dims);
    t.id_ = next_tensor_id();
    return t;
}

// ---- gradient API ------------------------------------------------------------------

void Tensor::set_requires_grad(bool r) {
    requires_grad_ = r;
    if (!r) grad_.reset();
}

void Tensor::backward(const Tensor *grad_output) { engine_backward(*this, grad_output); }

const Tensor *Tensor::grad_ref() const {
    if (grad_) return grad_.get();
    return accumulated_gradient(id_);
}

std::optional<Tensor> Tensor::grad_by_value() const {
    const Tensor *g = grad_ref();
    if (!g) return std::nullopt;
    return g->clone();  // utils.rs:525-534 returns a clone
}

void Tensor::set_grad(Tensor g) {
    if (requires_grad_) grad_ = std::make_shared<Tensor>(std::move(g));
}

void Tensor::accumulate_grad(Tensor g) {
    if (!requires_grad_) return;
    if (grad_) {
        Tensor acc = (defer_ok(size_) && grad_->size() == g.size()) ? map_binary(TS_HIP_MAP_ADD, *grad_, g)
                                                                     : same_shape(grad_->dev(), g.dev(), grad_->dims(), 0);
        grad_ = std::make_shared<Tensor>(std::move(acc));
    } else {
        grad_ = std::make_shared<Tensor>(std::move(g));
    }
}

// ---- recorded ops ---------------------------------------------------------------------

void Tensor::record(Tensor &out, std::vector<size_t> input_ids, GradFn fn) const {
    out.requires_grad_ = true;
    register_operation(out.id_, std::move(input_ids), std::move(fn));
}

// A deferred product [M, N] plus a row vector [N] (either order: fp32
// addition is commutative) becomes the product with a bias epilogue.
static bool fuse_bias(const Tensor &mat, const Tensor &vec) {
    const auto &a = mat.allocation();
    return fusion_enabled() && a && a->pending && a->pending->bare() && vec.allocation() &&
           is_row_broadcast(mat.dims(), vec.dims());
}

// A deferred product [M, N] (bare or with its bias) minus a same-shape
// tensor becomes the product with a subtraction in its store, where the
// narrow kernel takes the product (ts_hip_gemm_takes_sub).
static bool fuse_sub(const Tensor &mat, const Tensor &o) {
    const auto &a = mat.allocation();
    if (!fusion_enabled() || !a || !a->pending || !o.allocation() || mat.dims() != o.dims()) return false;
    const PendingGemm &p = *a->pending;
    return !p.src && !p.sub && !p.relu && !p.mask && a.get() != o.allocation().get() &&
           ts_hip_gemm_takes_sub(p.ta, p.tb, p.M, p.N, p.K) != 0;
}

Tensor Tensor::binary(const Tensor &o, GradFn::Kind kind) const {
    const bool same = dims_ == o.dims_;
    const int op = opcode(kind);
    Tensor out;
    const bool fuse_self = kind == GradFn::Kind::Add && fuse_bias(*this, o);
    const bool fuse_other = !fuse_self && kind == GradFn::Kind::Add && fuse_bias(o, *this);
    std::shared_ptr<PendingGemm> fused;
    if (kind == GradFn::Kind::Sub && fuse_sub(*this, o)) {
        out = new_uninit(dims_);
        fused = fork_pending(alloc_, out.alloc_);  // a record: fuse_sub found it pending
        fused->sub = o.alloc_;
        set_pending(out.alloc_, std::move(fused));
    } else if (fuse_self || fuse_other) {
        const Tensor &mat = fuse_self ? *this : o, &vec = fuse_self ? o : *this;
        out = new_uninit(mat.dims_);
        fused = fork_pending(mat.alloc_, out.alloc_);
        if (fused) {
            fused->bias = vec.alloc_;
            set_pending(out.alloc_, std::move(fused));
        } else {  // the product had a consumer already and has now run: the kernel reads it
            out = row_bcast(mat.dev(), vec.dev(), mat.dims_[0], mat.dims_[1], 0, fuse_other);
        }
    } else if (same && defer_ok(size_)) {  // deferred: the chain it belongs to runs as one pass
        static const uint8_t codes[4] = {TS_HIP_MAP_ADD, TS_HIP_MAP_SUB, TS_HIP_MAP_MUL, TS_HIP_MAP_DIV};
        out = map_binary(codes[op], *this, o, op == 3 ? TS_HIP_MAP_CHECKED : 0);
    } else if (same) {
        out = same_shape(dev(), o.dev(), dims_, op);
    } else if (is_row_broadcast(dims_, o.dims_)) {
        out = row_bcast(dev(), o.dev(), dims_[0], dims_[1], op, false);
    } else if (is_row_broadcast(o.dims_, dims_)) {
        out = row_bcast(o.dev(), dev(), o.dims_[0], o.dims_[1], op, true);
    } else {
        // broadcast_shapes (broadcasting.rs:362-407): materialise the operands
        // that need it, then the same-shape kernel
        const std::vector<size_t> full = broadcast_dims(dims_, o.dims_);
        Tensor ab, bb;
        const float *pa = dev(), *pb = o.dev();
        if (dims_ != full) {
            ab = bcast_to(dev(), dims_, full);
            pa = ab.dev();
        }
        if (o.dims_ != full) {
            bb = bcast_to(o.dev(), o.dims_, full);
            pb = bb.dev();
        }
        out = same_shape(pa, pb, full, op);
    }
    if ((requires_grad_ || o.requires_grad_) && is_grad_enabled()) {
        GradFn fn{kind};
        if (!same) {
            fn.has_shapes = true;
            fn.shape_a = dims_;
            fn.shape_b = o.dims_;
        }
        if (kind == GradFn::Kind::Mul || kind == GradFn::Kind::Div) fn.saved = {saved(), o.saved()};
        fn.req_left = requires_grad_;
        fn.req_right = o.requires_grad_;
        std::vector<size_t> ids;
        if (requires_grad_) ids.push_back(id_);
        if (o.requires_grad_) ids.push_back(o.id_);
        record(out, std::move(ids), std::move(fn));
    }
    return out;
}

Tensor Tensor::add_tensor(const Tensor &o) const { return binary(o, GradFn::Kind::Add); }
Tensor Tensor::sub_tensor(const Tensor &o) const { return binary(o, GradFn::Kind::Sub); }
Tensor Tensor::mul_tensor(const Tensor &o) const { return binary(o, GradFn::Kind::Mul); }
Tensor Tensor::div_tensor(const Tensor &o) const { return binary(o, GradFn::Kind::Div); }

Tensor Tensor::scalar_op(float s, GradFn::Kind kind) const {
    if (kind == GradFn::Kind::DivScalar && s == 0.0f)  // ops/div.rs:511-514
        throw Error("Division by zero: cannot divide tensor by zero scalar");
    Tensor out;
    if (defer_ok(size_)) {
        const uint8_t code = kind == GradFn::Kind::AddScalar   ? TS_HIP_MAP_ADD_S
                             : kind == GradFn::Kind::SubScalar ? TS_HIP_MAP_SUB_S
                             : kind == GradFn::Kind::MulScalar ? TS_HIP_MAP_MUL_S
                                                               : TS_HIP_MAP_DIV_S;
        out = map_unary(code, *this, s);
    } else {
        out = new_uninit(dims_);
    }
    if (!out.allocation() || !out.allocation()->map) launch(KernelClass::Elementwise, 8.0 * size_, "scalar op", [&] {
        switch (kind) {
            case GradFn::Kind::AddScalar: return ts_hip_add_scalar(dev(), s, out.dev_mut(), size_, S());
            case GradFn::Kind::SubScalar: return ts_hip_sub_scalar(dev(), s, out.dev_mut(), size_, S());
            case GradFn::Kind::MulScalar: return ts_hip_mul_scalar(dev(), s, out.dev_mut(), size_, S());
            default: return ts_hip_div_scalar(dev(), s, out.dev_mut(), size_, S());
        }
    });
    if (requires_grad_ && is_grad_enabled()) {
        GradFn fn{kind};
        fn.scalar = s;
        record(out, {id_}, std::move(fn));
    }
    return out;
}

Tensor Tensor::add_scalar(float s) const { return scalar_op(s, GradFn::Kind::AddScalar); }
Tensor Tensor::sub_scalar(float s) const { return scalar_op(s, GradFn::Kind::SubScalar); }
Tensor Tensor::mul_scalar(float s) const { return scalar_op(s, GradFn::Kind::MulScalar); }
Tensor Tensor::div_scalar(float s) const { return scalar_op(s, GradFn::Kind::DivScalar); }

Tensor Tensor::relu() const {
    Tensor out = new_uninit(dims_);
    std::shared_ptr<PendingGemm> fused;
    if (fusion_enabled() && alloc_ && alloc_->pending && !alloc_->pending->relu && !alloc_->pending->mask)
        fused = fork_pending(alloc_, out.alloc_);  // relu joins the deferred product
    if (fused) {
        fused->relu = true;
        set_pending(out.alloc_, std::move(fused));
    } else if (defer_ok(size_)) {
        out = map_unary(TS_HIP_MAP_RELU, *this);
    } else {
        launch(KernelClass::Elementwise, 8.0 * size_, "ts_hip_relu",
               [&] { return ts_hip_relu(dev(), out.dev_mut(), size_, S()); });
    }
    if (requires_grad_ && is_grad_enabled()) {
        GradFn fn{GradFn::Kind::Relu};
        // The reference saves its input (ops/relu.rs:80-87); the output has
        // the same sign test (relu(x) > 0 exactly when x > 0) and keeps the
        // input buffer free to be recycled.
        fn.saved = {out.saved()};
        record(out, {id_}, std::move(fn));
    }
    return out;
}

Tensor Tensor::pow_scalar(float e) const {
    Tensor out;
    if (e == 2.0f && defer_ok(size_)) {  // pow.rs:124-162: x * x
        out = map_unary(TS_HIP_MAP_SQUARE, *this);
    } else {
        out = new_uninit(dims_);
        launch(KernelClass::Elementwise, 8.0 * size_, "ts_hip_pow_scalar",
               [&] { return ts_hip_pow_scalar(dev(), e, out.dev_mut(), size_, S()); });
    }
    if (requires_grad_ && is_grad_enabled()) {
        GradFn fn{GradFn::Kind::PowScalar};
        fn.scalar = e;
        fn.saved = {saved()};
        record(out, {id_}, std::move(fn));
    }
    return out;
}

// A matrix operand as a product reads it: a 2-D transposed view (or copy)
// not yet written is its source read with the trans flag (transposes of the
// last two axes, transform/transpose.rs:283-291, are folded into the
// product's loads, never materialised); anything else as stored.
MatOperand mat_operand(const std::shared_ptr<Allocation> &a) {
    if (a && a->transpose && a->transpose->dims.size() == 2 && !a->pending && !a->map && !a->colsum)
        return {a->transpose->src, a->transpose->d0 != a->transpose->d1 ? 1 : 0};
    return {a, 0};
}

namespace {

// Output batch axes of batched_matmul (matmul/mod.rs:660-690): the batch
// axes (all but the last two) broadcast right-aligned.
std::vector<size_t> matmul_batch_dims(const std::vector<size_t> &a, const std::vector<size_t> &b) {
    const size_t ra = a.size() - 2, rb = b.size() - 2, r = ra > rb ? ra : rb;
    std::vector<size_t> out(r);
    for (size_t i = 0; i < r; ++i) {
        const size_t da = i < ra ? a[ra - 1 - i] : 1, db = i < rb ? b[rb - 1 - i] : 1;
        if (da == 1) out[r - 1 - i] = db;
        else if (db == 1 || da == db) out[r - 1 - i] = da;
        else throw Error("Cannot broadcast dimensions " + std::to_string(da) + " and " + std::to_string(db));
    }
    return out;
}

// Element strides of an operand's matrices along the output batch axes
// (calculate_batch_offset_with_broadcast, matmul/mod.rs:764-820): 0 where the
// operand has size 1 or lacks the axis.
std::vector<size_t> batch_strides(const std::vector<size_t> &dims, const std::vector<size_t> &out_batch) {
    const size_t nb = dims.size() - 2, q = out_batch.size();
    std::vector<size_t> st(q, 0);
    size_t stride = dims[nb] * dims[nb + 1];
    for (size_t j = nb; j-- > 0;) {
        st[j + (q - nb)] = dims[j] == 1 ? 0 : stride;
        stride *= dims[j];
    }
    return st;
}

// C[out_batch..., Mo, No] = op(A) . op(B) batch by batch; A and B carry their
// own (possibly broadcast) batch axes.
Tensor batched_gemm(int ta, int tb, const float *A, const std::vector<size_t> &adims, const float *B,
                    const std::vector<size_t> &bdims, const std::vector<size_t> &out_batch, size_t Mo, size_t No,
                    size_t Kc) {
    if (out_batch.size() > 6) throw Error("batched matmul supports up to 6 batch axes");
    std::vector<size_t> odims = out_batch;
    odims.push_back(Mo);
    odims.push_back(No);
    Tensor out = Tensor::new_uninit(odims);
    const std::vector<size_t> sa = batch_strides(adims, out_batch), sb = batch_strides(bdims, out_batch);
    const size_t lda = adims.back(), ldb = bdims.back();
    size_t batches = 1;
    for (size_t d : out_batch) batches *= d;
    if (out.size())
        launch(KernelClass::Gemm, 2.0 * Mo * No * Kc * batches, "ts_hip_gemm_batched", [&] {
            return ts_hip_gemm_batched(ta, tb, Mo, No, Kc, A, lda, B, ldb, out.dev_mut(), No, out_batch.size(),
                                       out_batch.data(), sa.data(), sb.data(), Mo * No, S());
        });
    return out;
}

Tensor gemv(int trans, const float *A, size_t rows, size_t cols, const float *x) {
    Tensor y = Tensor::new_uninit({trans ? cols : rows});
    const size_t ws = ts_hip_gemv_workspace_floats(trans, rows, cols);
    std::unique_ptr<Allocation> work = ws ? std::make_unique<Allocation>(ws) : nullptr;
    launch(trans ? KernelClass::Reduction : KernelClass::Elementwise, 4.0 * rows * cols + 4.0 * (rows + cols),
           "ts_hip_gemv", [&] {
               return ts_hip_gemv(trans, rows, cols, A, cols, x, y.dev_mut(), work ? work->get() : nullptr, ws, S());
           });
    return y;
}

Tensor outer(const float *a, size_t m, const float *b, size_t n) {
    Tensor out = Tensor::new_uninit({m, n});
    launch(KernelClass::Elementwise, 4.0 * (m * n + m + n), "ts_hip_outer",
           [&] { return ts_hip_outer(a, m, b, n, out.dev_mut(), S()); });
    return out;
}

}  // namespace

// ops/matmul/mod.rs:263-310: dispatch on the ranks -- 1D.1D dot, 1D.2D and
// 2D.1D vector products, 2D.2D, and batched N-D with broadcast batch axes.
Tensor Tensor::matmul(const Tensor &o) const {
    const size_t ra = dims_.size(), rb = o.dims_.size();
    Tensor out;
    if (ra == 1 && rb == 1) {  // dot_product_1d (:310-350): a scalar of shape []
        if (dims_[0] != o.dims_[0]) throw Error("Tensors must have same length for dot product");
        out = new_uninit({});
        const size_t ws = ts_hip_sum_workspace_floats(size_);
        Allocation work(ws);
        launch(KernelClass::Reduction, 8.0 * size_ + 4.0, "ts_hip_dot",
               [&] { return ts_hip_dot(dev(), o.dev(), size_, out.dev_mut(), work.get(), ws, S()); });
    } else if (ra == 1 && rb == 2) {  // vector_matrix_mult (:352-420)
        if (dims_[0] != o.dims_[0]) throw Error("Vector length must match matrix rows");
        out = gemv(1, o.dev(), o.dims_[0], o.dims_[1], dev());
    } else if (ra == 2 && rb == 1) {  // matrix_vector_mult (:488-560)
        if (dims_[1] != o.dims_[0]) throw Error("Matrix columns must match vector length");
        out = gemv(0, dev(), dims_[0], dims_[1], o.dev());
    } else if (ra == 2 && rb == 2) {  // matrix_matrix_mult (:572-611)
        const size_t m = dims_[0], k = dims_[1], n = o.dims_[1];
        if (k != o.dims_[0])
            throw Error("Inner dimensions must match: " + std::to_string(k) + " vs " + std::to_string(o.dims_[0]));
        out = new_uninit({m, n});
        // a transposed view is read as its source with the trans flag
        const MatOperand va = mat_operand(alloc_), vb = mat_operand(o.alloc_);
        const size_t lda = va.trans ? m : k, ldb = vb.trans ? k : n;
        if (fusion_enabled() && out.size_ && k) {  // deferred: a following bias add / relu joins it
            auto p = new_product(out.alloc_);
            p->ta = va.trans; p->tb = vb.trans;
            p->M = m; p->N = n; p->K = k; p->lda = lda; p->ldb = ldb;
            p->A = va.buf;
            p->B = vb.buf;
            set_pending(out.alloc_, std::move(p));
        } else if (out.size_) {
            const float *A = k ? va.buf->get() : nullptr, *B = k ? vb.buf->get() : nullptr;
            launch(KernelClass::Gemm, 2.0 * m * n * k, "ts_hip_gemm", [&] {
                return gemm2d(va.trans, vb.trans, m, n, k, A, lda, B, ldb, nullptr, false, nullptr, out.dev_mut(), n);
            });
        }
    } else {  // batched_matmul (:634-760)
        if (ra < 2 || rb < 2) throw Error("Batched matmul requires at least 2D tensors");
        const size_t m = dims_[ra - 2], k = dims_[ra - 1], k2 = o.dims_[rb - 2], n = o.dims_[rb - 1];
        if (k != k2)
            throw Error("Inner dimensions must match for batched matmul: " + std::to_string(k) + " vs " +
                        std::to_string(k2));
        out = batched_gemm(0, 0, dev(), dims_, o.dev(), o.dims_, matmul_batch_dims(dims_, o.dims_), m, n, k);
    }
    if ((requires_grad_ || o.requires_grad_) && is_grad_enabled()) {
        GradFn fn{GradFn::Kind::MatMul};
        fn.saved = {saved(), o.saved()};
        fn.req_left = requires_grad_;
        fn.req_right = o.requires_grad_;
        record(out, {id_, o.id_}, std::move(fn));  // matmul/mod.rs:303-306: always both
    }
    return out;
}

namespace {
// sum / mean of a deferred elementwise value in the pass that computes it
// (the bits of ts_hip_sum / ts_hip_mean over the stored values); the value
// itself is stored only when something besides its tensor holds it (a saved
// operand), else it stays deferred.  x is the tensor's own reference.
void fused_sum(const std::shared_ptr<Allocation> &x, float *out, bool mean) {
    MapBuilder b;
    b.p.n = x->map->n;
    const int r = b.import(*x->map, x);
    std::vector<MapOutput> outs;
    if (held_elsewhere(x, 1)) outs.push_back({x, r});
    else b.p.nodes[r].origin.reset();  // not stored: it stays deferred
    launch_program(b, outs, r, out, mean);
}

// Whether a sum of all n values of a, a deferred product, is deferred too:
// a weight-gradient product that reads a as its right operand (the README
// step's dW reads relu's output through relu's backward) then forms it in
// its own launch (ts_hip_gemm_colsum_bsum); otherwise it runs when read,
// with the same bits.  Only sums one workgroup covers.
bool sum_fits_product(const Allocation &a, size_t n) {
    constexpr size_t kOneWorkgroupSum = 16 * 1024;  // ts_hip_gemm_takes_bsum's limit
    return a.pending && !a.pending->src && n == a.pending->M * a.pending->N && n <= kOneWorkgroupSum;
}

// sum / mean of a deferred elementwise value or product, deferred in turn (x
// is the summed tensor's allocation); out reads x, so an in-place write of
// x's buffer runs it first
Tensor deferred_reduce(const std::shared_ptr<Allocation> &x, size_t n, bool mean) {
    Tensor out = Tensor::new_uninit({1});
    auto r = std::make_shared<PendingReduce>();
    r->x = x;
    r->n = n;
    r->mean = mean;
    add_reader(x, out.allocation());
    out.allocation()->reduce = std::move(r);
    pending_reduces().push_back(out.allocation());
    return out;
}
}  // namespace

void materialize_reduce(Allocation &a) {
    const std::shared_ptr<PendingReduce> r = a.reduce;
    float *out = a.raw();
    DevicePool::get().note_use(out);
    if (r->x->map && r->x->map->n == r->n) {
        fused_sum(r->x, out, r->mean);  // x's program with its sum; x stored only if held elsewhere
    } else {
        const float *x = r->x->get();
        const size_t ws = ts_hip_sum_workspace_floats(r->n);
        Allocation work(ws);
        launch(KernelClass::Reduction, 4.0 * r->n + 4.0, r->mean ? "ts_hip_mean" : "ts_hip_sum", [&] {
            return r->mean ? ts_hip_mean(x, r->n, out, work.get(), ws, S())
                           : ts_hip_sum(x, r->n, out, work.get(), ws, S());
        });
    }
    a.reduce.reset();
}

Tensor Tensor::sum() const {
    Tensor out;
    if (alloc_ && (alloc_->map || sum_fits_product(*alloc_, size_)) && fusion_enabled()) {
        out = deferred_reduce(alloc_, size_, false);
    } else {
        out = new_uninit({1});
        const size_t ws = ts_hip_sum_workspace_floats(size_);
        Allocation work(ws);
        launch(KernelClass::Reduction, 4.0 * size_ + 4.0, "ts_hip_sum",
               [&] { return ts_hip_sum(dev(), size_, out.dev_mut(), work.get(), ws, S()); });
    }
    if (requires_grad_) {  // reductions/sum.rs:131-138 (no is_grad_enabled check)
        GradFn fn{GradFn::Kind::ReduceSum};
        fn.input_shape = dims_;
        record(out, {id_}, std::move(fn));
    }
    return out;
}

Tensor Tensor::mean() const {
    Tensor out;
    if (alloc_ && (alloc_->map || sum_fits_product(*alloc_, size_)) && fusion_enabled()) {
        out = deferred_reduce(alloc_, size_, true);
    } else {
        out = new_uninit({1});
        const size_t ws = ts_hip_sum_workspace_floats(size_);
        Allocation work(ws);
        launch(KernelClass::Reduction, 4.0 * size_ + 4.0, "ts_hip_mean",
               [&] { return ts_hip_mean(dev(), size_, out.dev_mut(), work.get(), ws, S()); });
    }
    if (requires_grad_) {  // reductions/mean.rs:97-106
        GradFn fn{GradFn::Kind::ReduceMean};
        fn.input_shape = dims_;
        fn.numel = size_;
        record(out, {id_}, std::move(fn));
    }
    return out;
}

// ---- other recorded ops ---------------------------------------------------------------

// tensor/ops/{exp,log,sqrt,tanh,sigmoid,leaky_relu}.rs: out = f(self); recorded
// when self requires grad and grad is enabled, saving the output (exp, sqrt,
// tanh, sigmoid) or the input (log, leaky_relu).
template <class F>
Tensor Tensor::unary(GradFn::Kind kind, const char *what, bool save_output, float slope, F &&launcher) const {
    Tensor out = new_uninit(dims_);
    if (size_) launch(KernelClass::Elementwise, 8.0 * size_, what, [&] { return launcher(out.dev_mut()); });
    if (requires_grad_ && is_grad_enabled()) {
        GradFn fn{kind};
        fn.scalar = slope;
        fn.saved = {save_output ? out.saved() : saved()};
        record(out, {id_}, std::move(fn));
    }
    return out;
}

Tensor Tensor::exp() const {
    return unary(GradFn::Kind::Exp, "ts_hip_exp", true, 0.0f,
                 [&](float *o) { return ts_hip_exp(dev(), o, size_, S()); });
}
Tensor Tensor::log() const {
    return unary(GradFn::Kind::Log, "ts_hip_log", false, 0.0f,
                 [&](float *o) { return ts_hip_log(dev(), o, size_, S()); });
}
Tensor Tensor::sqrt() const {
    return unary(GradFn::Kind::Sqrt, "ts_hip_sqrt", true, 0.0f,
                 [&](float *o) { return ts_hip_sqrt(dev(), o, size_, S()); });
}
Tensor Tensor::tanh() const {
    return unary(GradFn::Kind::Tanh, "ts_hip_tanh", true, 0.0f,
                 [&](float *o) { return ts_hip_tanh(dev(), o, size_, S()); });
}
Tensor Tensor::sigmoid() const {
    return unary(GradFn::Kind::Sigmoid, "ts_hip_sigmoid", true, 0.0f,
                 [&](float *o) { return ts_hip_sigmoid(dev(), o, size_, S()); });
}
Tensor Tensor::leaky_relu(float slope) const {
    return unary(GradFn::Kind::LeakyRelu, "ts_hip_leaky_relu", false, slope,
                 [&](float *o) { return ts_hip_leaky_relu(dev(), slope, o, size_, S()); });
}

// softmax.rs:4-60
Tensor Tensor::softmax(size_t dim) const {
    if (dim >= dims_.size())
        throw Error("softmax dim " + std::to_string(dim) + " out of bounds for rank " + std::to_string(dims_.size()));
    size_t outer, reduce, inner;
    axis_view(dims_, dim, outer, reduce, inner);
    if (reduce == 0) throw Error("cannot softmax over empty dimension");
    Tensor out = new_uninit(dims_);
    if (size_)
        launch(KernelClass::Reduction, 8.0 * size_, "ts_hip_softmax",
               [&] { return ts_hip_softmax(dev(), out.dev_mut(), outer, reduce, inner, S()); });
    if (requires_grad_ && is_grad_enabled()) {
        GradFn fn{GradFn::Kind::Softmax};
        fn.axis = dim;
        fn.saved = {out.saved()};
        record(out, {id_}, std::move(fn));
    }
    return out;
}

namespace {

// sum_dims' output shape (reductions/sum.rs:237-252): reduced axes become 1
// (keepdim) or are dropped -- the reference drops every zero-size axis at this
// point -- and an empty shape becomes [1].
std::vector<size_t> sum_dims_shape(const std::vector<size_t> &in, const std::vector<size_t> &reduced, bool keepdim) {
    std::vector<size_t> out = in;
    for (size_t d : reduced) out[d] = keepdim ? 1 : 0;
    if (!keepdim) {
        std::vector<size_t> kept;
        for (size_t v : out)
            if (v != 0) kept.push_back(v);
        out = kept;
    }
    if (out.empty()) out.push_back(1);
    return out;
}

std::vector<size_t> checked_axes(const std::vector<size_t> &dims, size_t rank, const char *what) {
    if (dims.empty()) throw Error(std::string(what) + " requires at least one dimension");
    for (size_t d : dims)
        if (d >= rank)
            throw Error(std::string(what) + " dim " + std::to_string(d) + " out of bounds for rank " +
                        std::to_string(rank));
    std::vector<size_t> r = dims;
    std::sort(r.begin(), r.end());
    r.erase(std::unique(r.begin(), r.end()), r.end());
    return r;
}

unsigned axis_mask(const std::vector<size_t> &reduced) {
    unsigned m = 0;
    for (size_t d : reduced) m |= 1u << d;
    return m;
}

}  // namespace

Tensor Tensor::sum_dims(const std::vector<size_t> &dims, bool keepdim) const {
    const std::vector<size_t> reduced = checked_axes(dims, dims_.size(), "sum_dims");
    std::vector<size_t> out_dims = sum_dims_shape(dims_, reduced, keepdim);
    Tensor out = size_ ? reduce_axes(dev(), dims_, axis_mask(reduced), out_dims) : Tensor::zeros(out_dims);
    if (requires_grad_) {  // sum.rs:290-300 (no is_grad_enabled check)
        GradFn fn{GradFn::Kind::ReduceSumDims};
        fn.reduce_dims = reduced;
        fn.input_shape = dims_;
        fn.keepdim = keepdim;
        record(out, {id_}, std::move(fn));
    }
    return out;
}

// mean.rs:186-230: the sum times 1/factor, factor = product of the listed
// axes' sizes as given (a repeated axis counts twice, as there)
Tensor Tensor::mean_dims(const std::vector<size_t> &dims, bool keepdim) const {
    const std::vector<size_t> reduced = checked_axes(dims, dims_.size(), "mean_dims");
    size_t factor = 1;
    for (size_t d : dims) factor *= dims_[d];
    const float scale = factor > 0 ? 1.0f / static_cast<float>(factor) : 0.0f;
    std::vector<size_t> out_dims = sum_dims_shape(dims_, reduced, keepdim);
    Tensor out = size_ ? reduce_axes(dev(), dims_, axis_mask(reduced), out_dims, scale, true)
                       : Tensor::zeros(out_dims);
    if (requires_grad_) {
        GradFn fn{GradFn::Kind::ReduceMeanDims};
        fn.reduce_dims = reduced;
        fn.input_shape = dims_;
        fn.keepdim = keepdim;
        record(out, {id_}, std::move(fn));
    }
    return out;
}

// ---- host access ------------------------------------------------------------------------

void Tensor::copy_to_host(float *out, size_t len) const {
    if (len != size_)
        throw Error("copy_to_host: buffer of " + std::to_string(len) + " floats for a tensor of " +
                    std::to_string(size_));
    refuse_while_recording("copy_to_host");
    if (size_) check(ts_hip_memcpy_async(out, dev(), size_, 1, S()), "ts_hip_memcpy_async");
    Runtime::get().sync();
}

std::vector<float> Tensor::data() const {
    std::vector<float> h(size_);
    copy_to_host(h.data(), size_);
    return h;
}

float Tensor::value() const {
    if (size_ != 1)  // utils.rs:1251-1260
        throw Error("value() can only be called on tensors with exactly one element, got " +
                    std::to_string(size_));
    float v = 0.0f;
    copy_to_host(&v, 1);
    return v;
}

// ---- backward formulas ---------------------------------------------------------------------

std::vector<std::optional<Tensor>> GradFn::apply(const Tensor &go) const {
    using K = Kind;
    std::vector<std::optional<Tensor>> r;
    const size_t n = go.size();
    switch (kind) {
        case K::Add: {  // grad_fn/ops/add.rs:4-28
            if (!has_shapes) { r.emplace_back(go.alias()); r.emplace_back(go.alias()); }
            else { r.emplace_back(reduce_to(go, shape_a)); r.emplace_back(reduce_to(go, shape_b)); }
            break;
        }
        case K::Sub: {  // grad_fn/ops/sub.rs:4-33
            // Gradients go to the recorded inputs by position, and only the
            // inputs that require gradients are recorded: the second gradient
            // has a consumer only when both do (a loss y - t with constant
            // targets t skips the negation pass).
            const bool second = req_left && req_right;
            if (!has_shapes) {
                r.emplace_back(go.alias());
                if (second) r.emplace_back(neg_of(go));
            } else {
                r.emplace_back(reduce_to(go, shape_a));
                if (second) r.emplace_back(neg_of(reduce_to(go, shape_b)));
            }
            break;
        }
        case K::Mul: {  // grad_fn/ops/mul.rs:4-49
            // As for Sub: gradients go to the recorded inputs by position, so
            // the second one has a consumer only when both inputs are recorded.
            const SavedTensor &a = saved[0], &b = saved[1];
            const bool second = req_left && req_right;
            if (!has_shapes && defer_ok(n)) {  // deferred: joins the chain's pass
                r.emplace_back(map_binary(TS_HIP_MAP_MUL, go, Tensor::from_saved(b)));
                if (second) r.emplace_back(map_binary(TS_HIP_MAP_MUL, go, Tensor::from_saved(a)));
            } else if (!has_shapes) {
                Tensor ga = Tensor::new_uninit(go.dims());
                if (second) {
                    Tensor gb = Tensor::new_uninit(go.dims());
                    launch(KernelClass::Elementwise, 20.0 * n, "ts_hip_mul_backward", [&] {
                        return ts_hip_mul_backward(go.dev(), a.ptr(), b.ptr(), ga.dev_mut(), gb.dev_mut(), n, S());
                    });
                    r.emplace_back(std::move(ga));
                    r.emplace_back(std::move(gb));
                } else {
                    launch(KernelClass::Elementwise, 12.0 * n, "ts_hip_mul(grad)",
                           [&] { return ts_hip_mul(go.dev(), b.ptr(), ga.dev_mut(), n, S()); });
                    r.emplace_back(std::move(ga));
                }
            } else {
                r.emplace_back(reduce_to(with_bcast(go, b, 2), shape_a));
                if (second) r.emplace_back(reduce_to(with_bcast(go, a, 2), shape_b));
            }
            break;
        }
        case K::Div: {  // grad_fn/ops/div.rs:4-49
            const SavedTensor &a = saved[0], &b = saved[1];
            if (!has_shapes && req_left && req_right && defer_ok(n)) {  // deferred: joins the chain's pass
                // ga = go / b; gb = neg((go * a) / (b * b)); both divisions checked
                const Tensor ta = Tensor::from_saved(a), tb = Tensor::from_saved(b);
                r.emplace_back(map_binary(TS_HIP_MAP_DIV, go, tb, TS_HIP_MAP_CHECKED));
                auto p = defer(n, {{go.allocation(), false}, {ta.allocation(), false}, {tb.allocation(), false}},
                               [](MapBuilder &m, const std::vector<int> &v) {
                                   const int num = m.op(TS_HIP_MAP_MUL, v[0], v[1]);
                                   const int den = m.op(TS_HIP_MAP_MUL, v[2], v[2]);
                                   return m.op(TS_HIP_MAP_NEG, m.op(TS_HIP_MAP_DIV, num, den, 0.0f, TS_HIP_MAP_CHECKED), -1);
                               });
                r.emplace_back(deferred_tensor(go.dims(), std::move(p)));
            } else if (!has_shapes) {
                // the second gradient only when both inputs are recorded (see
                // Mul); the kernel still checks both divisors (b, then b*b)
                // for the reference's zero-divisor panic
                const bool second = req_left && req_right;
                Tensor ga = Tensor::new_uninit(go.dims());
                Tensor gb = second ? Tensor::new_uninit(go.dims()) : Tensor();
                launch(KernelClass::Elementwise, (second ? 20.0 : 16.0) * n, "ts_hip_div_backward", [&] {
                    return ts_hip_div_backward(go.dev(), a.ptr(), b.ptr(), ga.dev_mut(),
                                               second ? gb.dev_mut() : nullptr, n, tail8(n), tail32(n),
                                               Runtime::get().zero_index(), S());
                });
                r.emplace_back(std::move(ga));
                if (second) r.emplace_back(std::move(gb));
            } else {
                Tensor ga_full = with_bcast(go, b, 3);                  // go / b
                Tensor neg_grad = with_bcast(go, a, 2);                 // go * a
                Tensor b_sq = same_shape(b.ptr(), b.ptr(), b.dims, 2);  // b * b
                Tensor gb_full = with_bcast(neg_grad, b_sq.saved(), 3);
                Tensor gb_neg = neg_of(gb_full);
                r.emplace_back(reduce_to(ga_full, shape_a));
                r.emplace_back(reduce_to(gb_neg, shape_b));
            }
            break;
        }
        case K::AddScalar:
        case K::SubScalar:
            r.emplace_back(go.alias());
            break;
        case K::MulScalar:
        case K::DivScalar: {
            if (defer_ok(n)) {
                r.emplace_back(map_unary(kind == K::MulScalar ? TS_HIP_MAP_MUL_S : TS_HIP_MAP_DIV_S, go, scalar));
                break;
            }
            Tensor g = Tensor::new_uninit(go.dims());
            launch(KernelClass::Elementwise, 8.0 * n, "scalar grad", [&] {
                return kind == K::MulScalar ? ts_hip_mul_scalar(go.dev(), scalar, g.dev_mut(), n, S())
                                            : ts_hip_div_scalar(go.dev(), scalar, g.dev_mut(), n, S());
            });
            r.emplace_back(std::move(g));
            break;
        }
        case K::Relu: {  // grad_fn/ops/relu.rs:4-17 (saved[0] is the relu output)
            Tensor g = Tensor::new_uninit(go.dims());
            const auto &ga = go.allocation();
            std::shared_ptr<PendingGemm> fused;
            if (fusion_enabled() && ga && ga->pending && ga->pending->bare() && saved[0].alloc)
                fused = fork_pending(ga, g.allocation());  // the incoming gradient is a deferred dX product
            if (fused) {  // mask it in its store
                fused->mask = saved[0].alloc;
                set_pending(g.allocation(), std::move(fused));
            } else if (defer_ok(n) && saved[0].alloc) {
                g = map_binary(TS_HIP_MAP_RELU_BWD, Tensor::from_saved(saved[0]), go);
            } else {
                launch(KernelClass::Elementwise, 12.0 * n, "ts_hip_relu_backward", [&] {
                    return ts_hip_relu_backward(saved[0].ptr(), go.dev(), g.dev_mut(), n, S());
                });
            }
            r.emplace_back(std::move(g));
            break;
        }
        case K::PowScalar: {  // grad_fn/ops/pow.rs:5-27
            if (scalar == 2.0f && defer_ok(n)) {  // go * (2 * x): powf(x, 1) == x
                auto p = defer(n, {{go.allocation(), false}, {saved[0].alloc, false}},
                               [](MapBuilder &m, const std::vector<int> &v) {
                                   return m.op(TS_HIP_MAP_MUL, v[0], m.op(TS_HIP_MAP_MUL_S, v[1], -1, 2.0f));
                               });
                r.emplace_back(deferred_tensor(go.dims(), std::move(p)));
                break;
            }
            Tensor g = Tensor::new_uninit(go.dims());
            launch(KernelClass::Elementwise, 12.0 * n, "ts_hip_pow_backward", [&] {
                return ts_hip_pow_backward(saved[0].ptr(), go.dev(), g.dev_mut(), n, scalar, S());
            });
            r.emplace_back(std::move(g));
            break;
        }
        case K::MatMul: {  // grad_fn/ops/matmul.rs:4-219, transposes folded into the loads
            const SavedTensor &a = saved[0], &b = saved[1];
            const size_t ra = a.dims.size(), rb = b.dims.size();
            std::optional<Tensor> gl, gr;
            if (ra == 1 && rb == 1) {  // (1,1): go * b, go * a with the scalar go broadcast
                const size_t len = a.dims[0];
                Tensor gob = bcast_to(go.dev(), go.dims(), {len});
                if (req_left) gl = same_shape(gob.dev(), b.ptr(), {len}, 2);
                if (req_right) gr = same_shape(gob.dev(), a.ptr(), {len}, 2);
            } else if (ra == 1 && rb == 2) {  // (1,2): go . M^T, outer(v, go)
                if (req_left) gl = gemv(0, b.ptr(), b.dims[0], b.dims[1], go.dev());
                if (req_right) gr = outer(a.ptr(), a.dims[0], go.dev(), go.size());
            } else if (ra == 2 && rb == 1) {  // (2,1): outer(go, v), M^T . go
                if (req_left) gl = outer(go.dev(), go.size(), b.ptr(), b.dims[0]);
                if (req_right) gr = gemv(1, a.ptr(), a.dims[0], a.dims[1], go.dev());
            } else if (ra == 2 && rb == 2) {
                const size_t M = a.dims[0], Kd = a.dims[1], N = b.dims[1];
                // b (or a) a transposed view: its source, with the flag flipped
                const MatOperand va = mat_operand(a.alloc), vb = mat_operand(b.alloc);
                std::shared_ptr<PendingGemm> dx_pending;  // the dX product, when deferred
                if (req_left) {  // go[M,N] . b[Kd,N]^T -> [M,Kd]
                    Tensor t = Tensor::new_uninit({M, Kd});
                    const int tb = vb.trans ? 0 : 1;
                    const size_t ldb = vb.trans ? Kd : N;
                    if (fusion_enabled() && t.size() && N && go.allocation() && vb.buf) {
                        // deferred: relu's backward, usually next, joins it as a mask
                        auto p = new_product(t.allocation());
                        p->ta = 0; p->tb = tb;
                        p->M = M; p->N = Kd; p->K = N; p->lda = N; p->ldb = ldb;
                        p->A = go.allocation();
                        p->B = vb.buf;
                        dx_pending = p;
                        set_pending(t.allocation(), std::move(p));
                    } else {
                        const float *B = vb.buf ? vb.buf->get() : nullptr;
                        launch(KernelClass::Gemm, 2.0 * M * N * Kd, "ts_hip_gemm(dX)", [&] {
                            return gemm2d(0, tb, M, Kd, N, go.dev(), N, B, ldb, nullptr, false, nullptr,
                                          t.dev_mut(), Kd);
                        });
                    }
                    gl = std::move(t);
                }
                const int ta = va.trans ? 0 : 1;
                const size_t lda = va.trans ? M : Kd;
                const bool b_view = b.alloc && b.alloc->transpose && b.alloc->transpose->view;
                if (req_right && b_view && Kd && N && M && go.allocation() && va.buf) {
                    // b is a transposed view, so this gradient goes on through
                    // its Transpose: deferred, the product is then run with its
                    // operands swapped and writes the source's gradient directly
                    Tensor t = Tensor::new_uninit({Kd, N});
                    auto p = new_product(t.allocation());
                    p->ta = ta; p->tb = 0;
                    p->M = Kd; p->N = N; p->K = M; p->lda = lda; p->ldb = N;
                    p->A = va.buf;
                    p->B = go.allocation();
                    set_pending(t.allocation(), std::move(p));
                    gr = std::move(t);
                } else if (req_right) {  // a[M,Kd]^T . go[M,N] -> [Kd,N]
                    Tensor t = Tensor::new_uninit({Kd, N});
                    // A bias gradient still waiting to sum go's rows (the
                    // add before this product, grad_fn/ops/add.rs:4-28)
                    // comes out of this product: go is read once for both.
                    std::shared_ptr<Allocation> db;
                    if (fusion_enabled() && go.allocation())
                        for (auto &w : go.allocation()->readers) {
                            auto r = w.lock();
                            if (r && r->colsum && r->colsum->src == go.allocation() && r->colsum->rows == M &&
                                r->colsum->cols == N) {
                                db = r;
                                break;
                            }
                        }
                    // go deferred as a chain over one buffer (relu's backward of the
                    // seed, the MSE's gradient): the product reads that buffer and
                    // applies the chain as it loads it; go is never stored
                    ts_hip_operand_xf xb{};
                    std::shared_ptr<Allocation> leaf;
                    const bool fx = ts_hip_gemm_takes_xf(ta, 0, Kd, N, M, db ? 1 : 0) &&
                                    operand_xf(go.allocation(), leaf, xb);
                    // a deferred sum of the buffer read as B, or of a chain over
                    // it (the README step's loss over relu's output; an MSE's
                    // mean of d * d), comes out of this launch too
                    ts_hip_operand_xf xs{};
                    const std::shared_ptr<Allocation> bsum =
                        db && ts_hip_gemm_takes_bsum(ta, Kd, N, M)
                            ? pending_sum_of(fx ? leaf : go.allocation(), M * N, xs)
                            : nullptr;
                    const bool mean = bsum && bsum->reduce->mean;
                    if (db) db->colsum.reset();
                    if (bsum) bsum->reduce.reset();
                    // the launcher, from the buffers alone: run now, or held
                    // beside the deferred dX product (below)
                    const std::shared_ptr<Allocation> Ab = va.buf, Bb = fx ? leaf : go.allocation(),
                                                      out = t.allocation();
                    auto dw = [=]() {
                        const float *A = Ab ? Ab->get() : nullptr;
                        const float *B = Bb->get();
                        float *C = out->raw();
                        DevicePool::get().note_use(C);
                        if (bsum) {
                            float *sum = bsum->raw();
                            DevicePool::get().note_use(sum);
                            launch(KernelClass::Gemm, 2.0 * M * N * Kd, "ts_hip_gemm_colsum_bsum(dW, db, loss)", [&] {
                                return ts_hip_gemm_colsum_bsum(ta, Kd, N, M, A, lda, nullptr, B, fx ? &xb : nullptr, C,
                                                               N, db->raw(), xs.n_ops ? &xs : nullptr, sum,
                                                               mean ? 1 : 0, S());
                            });
                        } else if (db) {
                            const size_t ws = ts_hip_gemm_colsum_workspace_floats(ta, Kd, N, M);
                            std::unique_ptr<Allocation> work;  // from the pool: the launch allocates nothing
                            if (ws) work = std::make_unique<Allocation>(ws);
                            launch(KernelClass::Gemm, 2.0 * M * N * Kd, "ts_hip_gemm_colsum(dW, db)", [&] {
                                return ts_hip_gemm_colsum_xf(ta, Kd, N, M, A, lda, nullptr, B, N, fx ? &xb : nullptr,
                                                             C, N, db->raw(), work ? work->get() : nullptr, ws, S());
                            });
                        } else {
                            launch(KernelClass::Gemm, 2.0 * M * N * Kd, "ts_hip_gemm(dW)", [&] {
                                return gemm2d_xf(ta, 0, Kd, N, M, A, lda, nullptr, B, N, fx ? &xb : nullptr, nullptr,
                                                 false, nullptr, C, N);
                            });
                        }
                    };
                    // A layer with few outputs (N <= 16): dX (K = N, one k tile)
                    // and dW (the narrow kernel) are both latency-bound; dW is
                    // held until dX runs, and the two run as one launch.
                    if (dx_pending && N <= 16 && ts_hip_gemm_takes_sub(ta, 0, Kd, N, M)) {
                        auto sib = std::make_shared<SiblingLaunch>();
                        sib->run = dw;
                        sib->inputs = {Ab, Bb};
                        for (const auto &o : {out, db, bsum})
                            if (o) {
                                o->sibling = sib;
                                sib->outputs.push_back(o);
                            }
                        add_reader(Ab, out);  // an in-place write of an input runs it first
                        add_reader(Bb, out);
                        dx_pending->sibling = std::move(sib);
                    } else {
                        dw();
                    }
                    gr = std::move(t);
                }
            } else {  // batched (:150-219): go . B^T and A^T . go per batch, reduced to the operand shapes
                const size_t M = a.dims[ra - 2], Kd = a.dims[ra - 1], N = b.dims[rb - 1];
                const std::vector<size_t> ob = matmul_batch_dims(a.dims, b.dims);
                if (req_left)
                    gl = reduce_to(batched_gemm(0, 1, go.dev(), go.dims(), b.ptr(), b.dims, ob, M, Kd, N), a.dims);
                if (req_right)
                    gr = reduce_to(batched_gemm(1, 0, a.ptr(), a.dims, go.dev(), go.dims(), ob, Kd, N, M), b.dims);
            }
            r.emplace_back(std::move(gl));
            r.emplace_back(std::move(gr));
            break;
        }
        case K::Transpose:  // grad_fn/transforms/transpose.rs: the same two axes swapped back
            r.emplace_back(transposed_value(go, dim0, dim1, false));
            break;
        case K::Contiguous:  // grad_fn/mod.rs:534-537: the gradient passes through
            r.emplace_back(go.alias());
            break;
        case K::Exp: {  // grad_fn/ops/exp.rs: go * y
            Tensor g = Tensor::new_uninit(go.dims());
            launch(KernelClass::Elementwise, 12.0 * n, "exp grad",
                   [&] { return ts_hip_mul(go.dev(), saved[0].ptr(), g.dev_mut(), n, S()); });
            r.emplace_back(std::move(g));
            break;
        }
        case K::Log:
        case K::Sqrt:
        case K::Tanh:
        case K::Sigmoid:
        case K::LeakyRelu: {  // grad_fn/ops/{log,sqrt,tanh,sigmoid,leaky_relu}.rs
            Tensor g = Tensor::new_uninit(go.dims());
            launch(KernelClass::Elementwise, 12.0 * n, "activation grad", [&] {
                const float *sv = saved[0].ptr();
                switch (kind) {
                    case K::Log: return ts_hip_log_backward(sv, go.dev(), g.dev_mut(), n, S());
                    case K::Sqrt: return ts_hip_sqrt_backward(sv, go.dev(), g.dev_mut(), n, S());
                    case K::Tanh: return ts_hip_tanh_backward(sv, go.dev(), g.dev_mut(), n, S());
                    case K::Sigmoid: return ts_hip_sigmoid_backward(sv, go.dev(), g.dev_mut(), n, S());
                    default: return ts_hip_leaky_relu_backward(sv, go.dev(), g.dev_mut(), n, scalar, S());
                }
            });
            r.emplace_back(std::move(g));
            break;
        }
        case K::Softmax: {  // grad_fn/ops/softmax.rs:4-38
            size_t outer, red, inner;
            axis_view(saved[0].dims, axis, outer, red, inner);
            Tensor g = Tensor::new_uninit(go.dims());
            launch(KernelClass::Reduction, 12.0 * n, "ts_hip_softmax_backward", [&] {
                return ts_hip_softmax_backward(saved[0].ptr(), go.dev(), g.dev_mut(), outer, red, inner, S());
            });
            r.emplace_back(std::move(g));
            break;
        }
        case K::ReduceSumDims:
        case K::ReduceMeanDims: {  // grad_fn/reductions/sum.rs:18-52, mean.rs:32-52
            // go holds the keepdim layout's values: broadcast them back over the
            // reduced axes (times 1/factor for the mean, factor over the
            // deduplicated axes as the backward computes it)
            std::vector<size_t> kd = input_shape;
            size_t factor = 1;
            for (size_t d : reduce_dims) {
                kd[d] = 1;
                factor *= input_shape[d];
            }
            const bool mean = kind == K::ReduceMeanDims;
            const float scale = factor > 0 ? 1.0f / static_cast<float>(factor) : 0.0f;
            if (product(input_shape) && go.size() != product(kd))
                throw Error("reduce_dims backward: gradient of " + std::to_string(go.size()) +
                            " elements for an output of " + std::to_string(product(kd)));
            r.emplace_back(bcast_to(go.dev(), kd, input_shape, scale, mean));
            break;
        }
        case K::ReduceSum: {  // grad_fn/reductions/sum.rs:4-16
            if (go.size() == 1 && defer_ok(product(input_shape))) {  // every element takes go[0]
                auto p = defer(product(input_shape), {{go.allocation(), true}},
                               [](MapBuilder &, const std::vector<int> &v) { return v[0]; });
                r.emplace_back(deferred_tensor(input_shape, std::move(p)));
                break;
            }
            Tensor g = Tensor::new_uninit(input_shape);
            launch(KernelClass::Elementwise, 4.0 * g.size(), "sum grad", [&] {
                return go.size() == 1 ? ts_hip_fill_from_device(g.dev_mut(), go.dev(), 1.0f, 0, g.size(), S())
                                      : ts_hip_fill(g.dev_mut(), 1.0f, g.size(), S());
            });
            r.emplace_back(std::move(g));
            break;
        }
        case K::ReduceMean: {  // grad_fn/reductions/mean.rs:4-30
            const float base = numel > 0 ? 1.0f / static_cast<float>(numel) : 0.0f;
            if (go.size() == 1 && defer_ok(product(input_shape))) {  // base * go[0] (one product, commutative)
                auto p = defer(product(input_shape), {{go.allocation(), true}},
                               [&](MapBuilder &m, const std::vector<int> &v) {
                                   return m.op(TS_HIP_MAP_MUL_S, v[0], -1, base);
                               });
                r.emplace_back(deferred_tensor(input_shape, std::move(p)));
                break;
            }
            Tensor g = Tensor::new_uninit(input_shape);
            launch(KernelClass::Elementwise, 4.0 * g.size(), "mean grad", [&] {
                return go.size() == 1 ? ts_hip_fill_from_device(g.dev_mut(), go.dev(), base, 1, g.size(), S())
                                      : ts_hip_fill(g.dev_mut(), base, g.size(), S());
            });
            r.emplace_back(std::move(g));
            break;
        }
    }
    return r;
}

}  // namespace ts
