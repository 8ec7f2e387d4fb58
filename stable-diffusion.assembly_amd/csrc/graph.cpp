// The graph side of the hooks, without ggml: which node this library takes,
// the chain of nodes after it that it computes along with it, and the
// computation of both -- the decisions of sdasm_compute_nodes and
// sdasm_work_size (hooks.cc:29-196) and of match_chain, redirect_apart and
// match_gated_gelu (fusion.cc:100-394), made over plain node descriptors
// (sdhip_node) that a ggml backend fills from its graph (an adapter that
// mirrors each ggml_tensor into one sdhip_node a graph), so
// that the same nodes are fused, and the same redirects taken, as the
// reference fuses and takes them.

#include <hip/hip_runtime.h>

#include <cstring>

#include "../../include/sdhip.h"
#include "host.h"

namespace sdhip {

namespace {

// Whether the bytes of two tensors share any (memory.cc:42-55): addresses
// compared, never read.
bool overlap(const sdhip_tensor &a, const sdhip_tensor &b) {
    const size_t an = tensor_span(&a), bn = tensor_span(&b);
    if (a.data == nullptr || b.data == nullptr || an == 0 || bn == 0) return false;
    return spans_overlap(a.data, an, b.data, bn);
}

// holds<float> (memory.h:196-209): single precision, aligned, whole strides.
bool holds_float(const sdhip_tensor &t) {
    if (t.type != SDHIP_TYPE_F32 || (reinterpret_cast<uintptr_t>(t.data) & 3) != 0) return false;
    for (int k = 0; k < 4; ++k) {
        if (t.nb[k] % 4 != 0) return false;
    }
    return true;
}

bool shape_of(const sdhip_tensor &a, const sdhip_tensor &b) {
    for (int k = 0; k < 4; ++k) {
        if (a.ne[k] != b.ne[k]) return false;
    }
    return true;
}

// fusion.cc:29-35: the same extents, strides, memory and type.
bool layout_of(const sdhip_tensor &a, const sdhip_tensor &b) {
    for (int k = 0; k < 4; ++k) {
        if (a.ne[k] != b.ne[k] || a.nb[k] != b.nb[k]) return false;
    }
    return a.data == b.data && a.type == b.type;
}

// ggml_is_contiguous.
bool dense(const sdhip_tensor &t) {
    const int64_t size = t.type == SDHIP_TYPE_F16 ? 2 : 4;
    return t.nb[0] == size && t.nb[1] == t.nb[0] * t.ne[0] && t.nb[2] == t.nb[1] * t.ne[1] &&
           t.nb[3] == t.nb[2] * t.ne[2];
}

// ggml_op_is_empty: the nodes that only describe other nodes' memory.
bool empty_op(int32_t op) {
    return op == SDHIP_OP_NONE || op == SDHIP_OP_VIEW || op == SDHIP_OP_RESHAPE || op == SDHIP_OP_PERMUTE ||
           op == SDHIP_OP_TRANSPOSE;
}

bool computed(const sdhip_node *n) { return (n->flags & SDHIP_FLAG_COMPUTE) != 0; }
bool graph_output(const sdhip_node *n) { return (n->flags & SDHIP_FLAG_OUTPUT) != 0; }

float param_float(const sdhip_node *n, int i) {
    float f;
    std::memcpy(&f, &n->op_params[i], sizeof f);
    return f;
}

const sdhip_tensor *src_tensor(const sdhip_node *n, int i) {
    return n->src[i] != nullptr ? &n->src[i]->tensor : nullptr;
}

// Which operation a node is computed as here, or SDHIP_OP_NONE (hooks.cc:29-55).
int32_t taken(const sdhip_node *n) {
    const sdhip_tensor *y = &n->tensor;
    switch (n->op) {
    case SDHIP_OP_CONV_2D:
        return src_tensor(n, 0) != nullptr && src_tensor(n, 1) != nullptr &&
                       sdhip_conv2d_supported(src_tensor(n, 0), src_tensor(n, 1), y, n->op_params)
                   ? SDHIP_OP_CONV_2D
                   : SDHIP_OP_NONE;
    case SDHIP_OP_MUL_MAT:
        return sdhip_mul_mat_supported(src_tensor(n, 0), src_tensor(n, 1), y) ? SDHIP_OP_MUL_MAT : SDHIP_OP_NONE;
    case SDHIP_OP_FLASH_ATTN_EXT:
        // No mask (src[3]) and no sinks (src[4]).
        return n->src[3] == nullptr && n->src[4] == nullptr &&
                       sdhip_attention_supported(src_tensor(n, 0), src_tensor(n, 1), src_tensor(n, 2), y,
                                                 param_float(n, 1), param_float(n, 2))
                   ? SDHIP_OP_FLASH_ATTN_EXT
                   : SDHIP_OP_NONE;
    case SDHIP_OP_GROUP_NORM:
        return sdhip_group_norm_supported(src_tensor(n, 0), y, n->op_params[0]) ? SDHIP_OP_GROUP_NORM
                                                                                 : SDHIP_OP_NONE;
    case SDHIP_OP_NORM:
        return sdhip_norm_supported(src_tensor(n, 0), y) ? SDHIP_OP_NORM : SDHIP_OP_NONE;
    default:
        return SDHIP_OP_NONE;
    }
}

// A chain as match_chain builds it (fusion.h:63-108): the steps in the C
// ABI's form, each step's operand node, the last node, the redirect's node.
struct Chain {
    sdhip_epilogue e{};
    const sdhip_node *operands[SDHIP_MAX_STEPS] = {};
    int last_node = -1;
    const sdhip_node *redirect = nullptr;

    bool empty() const { return e.count == 0 && e.from_redirect == 0; }
};

void add_step(Chain &c, int32_t kind, const sdhip_node *operand) {
    sdhip_step &s = c.e.steps[c.e.count];
    s = sdhip_step{};
    s.kind = kind;
    if (operand != nullptr) s.operand = operand->tensor;
    c.operands[c.e.count] = operand;
    ++c.e.count;
}

// Whether node `from` or any after it reads one of `tensors`, or a view of
// one (fusion.cc:315-330).
bool read_after(const sdhip_node *const *nodes, int n_nodes, int from, const sdhip_node *const *tensors, int count) {
    for (int i = from; i < n_nodes; ++i) {
        for (const sdhip_node *s : nodes[i]->src) {
            for (const sdhip_node *t = s; t != nullptr; t = t->view_src) {
                for (int u = 0; u < count; ++u) {
                    if (t == tensors[u]) return true;
                }
            }
        }
    }
    return false;
}

constexpr int kMaxUnwritten = SDHIP_MAX_STEPS + 8;

// fusion.cc:136-270.
Chain match_chain(const sdhip_node *const *nodes, int n_nodes, int index, bool silu, bool positions, bool redirect) {
    Chain c;
    const sdhip_node *head = nodes[index];
    const sdhip_tensor &ht = head->tensor;
    c.last_node = index;
    if (!holds_float(ht) || ht.nb[0] != 4) return c;
    int j = index + 1;
    for (; j < n_nodes && c.e.count < SDHIP_MAX_STEPS; ++j) {
        const sdhip_node *node = nodes[j];
        if (empty_op(node->op)) continue;
        if (!computed(node) || !layout_of(node->tensor, ht)) break;
        if (node->op == SDHIP_OP_UNARY && node->unary == SDHIP_UNARY_SILU && silu && node->src[0] != nullptr &&
            node->src[0]->tensor.data == ht.data) {
            add_step(c, SDHIP_STEP_SILU, nullptr);
            c.last_node = j;
            continue;
        }
        if (node->op != SDHIP_OP_ADD && node->op != SDHIP_OP_MUL) break;
        const sdhip_node *a = node->src[0];
        const sdhip_node *b = node->src[1];
        if (a == nullptr || b == nullptr) break;
        // An in-place ADD or MUL updates its first source, so the step is
        // ours only if that source is the head's memory, unchanged in shape;
        // the second source is the step's operand.
        const sdhip_tensor &bt = b->tensor;
        if (a->tensor.data != ht.data || !shape_of(a->tensor, ht) || overlap(bt, ht) || !holds_float(bt) ||
            bt.nb[0] != 4) {
            break;
        }
        bool fits = true;
        int64_t nb[4];
        for (int k = 0; k < 4; ++k) {
            if (bt.ne[k] != ht.ne[k] && bt.ne[k] != 1) fits = false;
            nb[k] = bt.ne[k] == 1 ? 0 : bt.nb[k] / 4;
        }
        if (positions) {
            // The convolution's epilogue walks an image's positions as one
            // flat run, so within a channel the operand must either be a
            // single number or laid out row by row exactly like the output.
            const bool broadcast = nb[0] == 0 && nb[1] == 0;
            const bool rows = nb[0] == 1 && nb[1] == ht.ne[0];
            fits = fits && (broadcast || rows);
        }
        if (!fits) break;
        add_step(c, node->op == SDHIP_OP_ADD ? SDHIP_STEP_ADD : SDHIP_STEP_MUL, b);
        c.last_node = j;
    }
    // A skip connection after the chain: skipping view-only nodes, the next
    // node may add the head's tensor to a same-shaped, same-strided tensor
    // and write the sum somewhere else.  That sum can be written directly.
    for (; redirect && j < n_nodes && empty_op(nodes[j]->op); ++j) {
    }
    if (!redirect || j >= n_nodes || c.e.count >= SDHIP_MAX_STEPS) return c;
    const sdhip_node *node = nodes[j];
    const auto alike = [&](const sdhip_node *t) {
        if (t == nullptr || !holds_float(t->tensor)) return false;
        for (int k = 0; k < 4; ++k) {
            if (t->tensor.ne[k] != ht.ne[k] || t->tensor.nb[k] != ht.nb[k]) return false;
        }
        return true;
    };
    if (node->op != SDHIP_OP_ADD || !computed(node) || !alike(node) || node->tensor.data == ht.data) return c;
    const sdhip_node *a = node->src[0];
    const sdhip_node *b = node->src[1];
    const sdhip_node *other = a != nullptr && a->tensor.data == ht.data && alike(a)   ? b
                              : b != nullptr && b->tensor.data == ht.data && alike(b) ? a
                                                                                      : nullptr;
    if (!alike(other) || overlap(other->tensor, ht)) return c;
    // Writing the sum directly means the head's own tensor, and every chain
    // node living in its memory, is never written.  That is only allowed if
    // none of them is a graph output and no later node reads one of them.
    // Too many of them to track: no redirect.
    const sdhip_node *unwritten[kMaxUnwritten];
    int count = 0;
    for (int i = index; i <= c.last_node; ++i) {
        const sdhip_node *t = nodes[i];
        if (t->tensor.data != ht.data) continue;
        if (graph_output(t) || count == kMaxUnwritten) return c;
        unwritten[count++] = t;
    }
    if (read_after(nodes, n_nodes, j + 1, unwritten, count)) return c;
    if (other->tensor.data == node->tensor.data) {
        // The skip tensor is the destination itself, so the epilogue starts
        // its sum from the value already there.  That moves the skip term to
        // the front of the sum, which is only the same sum in the reference's
        // rounding order when every earlier step is an addition.
        for (int s = 0; s < c.e.count; ++s) {
            if (c.e.steps[s].kind != SDHIP_STEP_ADD) return c;
        }
        c.e.from_redirect = 1;
        c.last_node = j;
        c.redirect = node;
        return c;
    }
    add_step(c, SDHIP_STEP_ADD, other);
    c.last_node = j;
    c.redirect = node;
    return c;
}

// fusion.cc:272-288: what the redirect writes is none of what the operation
// or the chain reads.
bool redirect_apart(const sdhip_node *node, const Chain &c) {
    if (c.redirect == nullptr) return true;
    const sdhip_tensor &out = c.redirect->tensor;
    for (const sdhip_node *s : node->src) {
        if (s != nullptr && s->tensor.data != nullptr && overlap(out, s->tensor)) return false;
    }
    for (int i = 0; i < c.e.count; ++i) {
        if (c.operands[i] != nullptr && overlap(out, c.operands[i]->tensor)) return false;
    }
    return true;
}

// fusion.cc:333-345: whether `view` selects exactly the columns [begin,
// begin + width) of `whole`, keeping each of its rows and their strides.
bool columns_of(const sdhip_node *view, const sdhip_node *whole, int64_t begin, int64_t width) {
    const sdhip_tensor &v = view->tensor, &w = whole->tensor;
    if (!holds_float(v) || !holds_float(w) || v.ne[0] != width || v.nb[0] != 4 || begin > w.ne[0] ||
        reinterpret_cast<uintptr_t>(v.data) != address_past(w.data, begin * w.nb[0])) {
        return false;
    }
    for (int k = 1; k < 4; ++k) {
        if (v.ne[k] != w.ne[k] || v.nb[k] != w.nb[k]) return false;
    }
    return true;
}

struct Gated {
    const sdhip_node *out = nullptr;
    int last_node = -1;
};

// fusion.cc:347-394: VIEW, VIEW, CONT (the gate), GELU in place, MUL.
Gated match_gated_gelu(const sdhip_node *const *nodes, int n_nodes, int index, const Chain &c) {
    Gated r;
    const int j = c.last_node + 1;
    if (j + 5 > n_nodes) return r;
    const sdhip_node *head = nodes[index];
    const sdhip_node *v0 = nodes[j];
    const sdhip_node *v1 = nodes[j + 1];
    const sdhip_node *cont = nodes[j + 2];
    const sdhip_node *gelu = nodes[j + 3];
    const sdhip_node *mul = nodes[j + 4];
    if (head->tensor.type != SDHIP_TYPE_F32 || !dense(head->tensor) || head->tensor.ne[0] % 2 != 0 ||
        v0->op != SDHIP_OP_VIEW || v1->op != SDHIP_OP_VIEW || cont->op != SDHIP_OP_CONT ||
        gelu->op != SDHIP_OP_UNARY || gelu->unary != SDHIP_UNARY_GELU || mul->op != SDHIP_OP_MUL) {
        return r;
    }
    const sdhip_node *gate = cont->src[0];
    const sdhip_node *x = gate == v0 ? v1 : gate == v1 ? v0 : nullptr;
    const int64_t half = head->tensor.ne[0] / 2;
    if (x == nullptr || !columns_of(x, head, 0, half) || !columns_of(gate, head, half, half) ||
        gelu->src[0] != cont || gelu->tensor.data != cont->tensor.data || mul->src[0] != x || mul->src[1] != gelu ||
        mul->tensor.type != SDHIP_TYPE_F32 || !dense(mul->tensor) || !shape_of(mul->tensor, x->tensor)) {
        return r;
    }
    // The fused form writes only the MUL's output, so the product, its chain
    // and the four nodes of the pattern are never written: none may be a
    // graph output or be read later.  Too many of them to track: no match.
    if (c.last_node - index + 1 > kMaxUnwritten) return r;
    const sdhip_node *unwritten[kMaxUnwritten + 4];
    int count = 0;
    for (int i = index; i <= c.last_node; ++i) unwritten[count++] = nodes[i];
    for (const sdhip_node *t : {v0, v1, cont, gelu}) unwritten[count++] = t;
    for (int i = 0; i < count; ++i) {
        if (graph_output(unwritten[i])) return r;
    }
    if (read_after(nodes, n_nodes, j + 5, unwritten, count)) return r;
    r.out = mul;
    r.last_node = j + 4;
    return r;
}

// mul_mat_gated_supported (mul_mat.cc:1128-1151): the gated output overlaps
// none of the chain's operands either.
bool gated_taken(const sdhip_node *node, const Chain &c, const sdhip_node *out) {
    if (!sdhip_mul_mat_gated_supported(src_tensor(node, 0), src_tensor(node, 1), &node->tensor, &out->tensor)) {
        return false;
    }
    for (int i = 0; i < c.e.count; ++i) {
        if (c.operands[i] != nullptr && overlap(out->tensor, c.operands[i]->tensor)) return false;
    }
    return true;
}

// The node's plan: hooks.cc:100-147.
void plan(const sdhip_node *const *nodes, int n_nodes, int index, sdhip_node_plan &p) {
    std::memset(&p, 0, sizeof p);
    const sdhip_node *node = nodes[index];
    const int32_t op = taken(node);
    p.taken = op;
    if (op == SDHIP_OP_NONE) return;
    Chain chain;
    chain.last_node = index;
    Gated gated;
    const Tuning &t = tuning();
    if (t.fuse != 0) {
        switch (op) {
        case SDHIP_OP_CONV_2D:
        case SDHIP_OP_MUL_MAT: {
            const bool positions = op == SDHIP_OP_CONV_2D;
            chain = match_chain(nodes, n_nodes, index, false, positions, t.fuse_residual != 0);
            if (!redirect_apart(node, chain)) chain = match_chain(nodes, n_nodes, index, false, positions, false);
            if (op == SDHIP_OP_MUL_MAT && chain.redirect == nullptr) {
                gated = match_gated_gelu(nodes, n_nodes, index, chain);
                if (gated.out != nullptr && !gated_taken(node, chain, gated.out)) gated = Gated{};
            }
            break;
        }
        case SDHIP_OP_GROUP_NORM:
        case SDHIP_OP_NORM:
            chain = match_chain(nodes, n_nodes, index, true, false, false);
            break;
        default:
            break;
        }
    }
    p.chain = chain.e;
    p.chain.redirect = chain.redirect != nullptr ? &chain.redirect->tensor : nullptr;
    p.gated_out = gated.out;
    if (gated.out != nullptr) {
        p.count = gated.last_node - index + 1;
    } else if (op == SDHIP_OP_FLASH_ATTN_EXT || chain.empty()) {
        p.count = 1;
    } else {
        p.count = chain.last_node - index + 1;
    }
}

}  // namespace

}  // namespace sdhip

using namespace sdhip;

extern "C" {

sdhip_status sdhip_plan_nodes(const sdhip_node *const *nodes, int n_nodes, int index, sdhip_node_plan *p) {
    if (p == nullptr) return fail(SDHIP_ERROR, "plan_nodes: no plan to fill");
    std::memset(p, 0, sizeof *p);
    if (nodes == nullptr || n_nodes <= 0 || index < 0 || index >= n_nodes || nodes[index] == nullptr) {
        return fail(SDHIP_UNSUPPORTED, "plan_nodes: no node %d of %d", index, n_nodes);
    }
    for (int i = 0; i < n_nodes; ++i) {
        if (nodes[i] == nullptr) return fail(SDHIP_ERROR, "plan_nodes: node %d is null", i);
    }
    plan(nodes, n_nodes, index, *p);
    return p->taken == SDHIP_OP_NONE ? fail(SDHIP_UNSUPPORTED, "plan_nodes: node %d not taken", index) : SDHIP_OK;
}

int sdhip_node_work_size(const sdhip_node *node, size_t *size) {
    if (node == nullptr || size == nullptr) return 0;
    const sdhip_tensor *y = &node->tensor;
    switch (taken(node)) {
    case SDHIP_OP_CONV_2D:
        *size = sdhip_conv2d_work_size(src_tensor(node, 0), src_tensor(node, 1), y, node->op_params);
        return 1;
    case SDHIP_OP_MUL_MAT:
        *size = sdhip_mul_mat_work_size(src_tensor(node, 0), src_tensor(node, 1), y);
        return 1;
    case SDHIP_OP_FLASH_ATTN_EXT:
        *size = sdhip_attention_work_size(src_tensor(node, 0), src_tensor(node, 1), src_tensor(node, 2), y);
        return 1;
    case SDHIP_OP_GROUP_NORM:
        *size = sdhip_group_norm_work_size(src_tensor(node, 0), y, node->op_params[0]);
        return 1;
    case SDHIP_OP_NORM:
        *size = 0;
        return 1;
    default:
        return 0;
    }
}

int sdhip_compute_nodes(const sdhip_node *const *nodes, int n_nodes, int index, void *work, size_t work_size,
                        void *stream) {
    if (nodes == nullptr || n_nodes <= 0 || index < 0 || index >= n_nodes || nodes[index] == nullptr) return 0;
    const sdhip_node *node = nodes[index];
    // What the node writes was derived from nothing that is kept, or is not
    // to be kept any more, whoever computes it (hooks.cc:104-108).
    if (node->tensor.data != nullptr) sdhip_forget(node->tensor.data, tensor_span(&node->tensor));
    sdhip_node_plan p;
    const sdhip_status planned = sdhip_plan_nodes(nodes, n_nodes, index, &p);
    if (planned == SDHIP_UNSUPPORTED) return 0;
    if (planned != SDHIP_OK) return -1;
    // And what a fused node writes in place of the node's own (hooks.cc:110-121).
    const sdhip_tensor *written[] = {p.chain.redirect, p.gated_out != nullptr ? &p.gated_out->tensor : nullptr};
    for (const sdhip_tensor *t : written) {
        if (t != nullptr && t->data != nullptr) sdhip_forget(t->data, tensor_span(t));
    }
    const sdhip_tensor *y = &node->tensor;
    const sdhip_epilogue *chain = p.chain.count > 0 || p.chain.redirect != nullptr ? &p.chain : nullptr;
    sdhip_status s = SDHIP_ERROR;
    switch (p.taken) {
    case SDHIP_OP_CONV_2D:
        s = sdhip_conv2d(src_tensor(node, 0), src_tensor(node, 1), y, node->op_params, chain, work, work_size,
                         stream);
        break;
    case SDHIP_OP_MUL_MAT:
        s = p.gated_out != nullptr
                ? sdhip_mul_mat_gated(src_tensor(node, 0), src_tensor(node, 1), y, chain, &p.gated_out->tensor, work,
                                      work_size, stream)
                : sdhip_mul_mat(src_tensor(node, 0), src_tensor(node, 1), y, chain, work, work_size, stream);
        break;
    case SDHIP_OP_FLASH_ATTN_EXT:
        s = sdhip_attention(src_tensor(node, 0), src_tensor(node, 1), src_tensor(node, 2), y, param_float(node, 0),
                            param_float(node, 1), param_float(node, 2), work, work_size, stream);
        break;
    case SDHIP_OP_GROUP_NORM:
        s = sdhip_group_norm(src_tensor(node, 0), y, node->op_params[0], param_float(node, 1), chain, work,
                             work_size, stream);
        break;
    case SDHIP_OP_NORM:
        s = sdhip_norm(src_tensor(node, 0), y, param_float(node, 0), chain, stream);
        break;
    default:
        break;
    }
    return s == SDHIP_OK ? p.count : -1;
}

}  // extern "C"
