// The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer:
// every entry point that reads descriptors only -- the operations'
// predicates, work sizes and path choice, the graph planner, the tuning's
// parser, ToDo's step -- driven with randomized descriptors, graphs and
// tuning strings, ggml-shaped where ggml guarantees a shape (an operation's
// sources present) and arbitrary elsewhere (extents, strides, types, null
// data, parameters).  What each call answers is checked by the Python tests;
// here any out-of-bounds access, use of freed memory, overflow or other
// undefined behaviour stops the run.  No GPU is touched.
//
//   make -C stable-diffusion.assembly_amd host_check && stable-diffusion.assembly_amd/_build/host_check [cases [seed]]

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "../include/sdhip.h"

// The HIP runtime's own allocations live until the process ends.
extern "C" const char *__asan_default_options() { return "detect_leaks=0"; }

namespace {

std::mt19937_64 rng(12345);

int64_t pick(std::initializer_list<int64_t> values) {
    const size_t i = rng() % values.size();
    return *(values.begin() + i);
}

int64_t extent() { return pick({0, 1, 1, 1, 2, 3, 4, 7, 8, 9, 16, 31, 32, 40, 64, 77, 80, 128, 160, 300, 320, 1024}); }

// Host memory the descriptors point into: never read by the calls here.
std::vector<char> arena(1 << 16);

sdhip_tensor tensor() {
    sdhip_tensor t{};
    t.type = static_cast<int32_t>(pick({0, 0, 0, 1, 1, 2, -1}));
    for (int i = 0; i < 4; ++i) t.ne[i] = extent();
    const int64_t size = t.type == 1 ? 2 : 4;
    switch (rng() % 4) {
    case 0:  // contiguous
    case 1:
        t.nb[0] = size;
        for (int i = 1; i < 4; ++i) t.nb[i] = t.nb[i - 1] * (t.ne[i - 1] > 0 ? t.ne[i - 1] : 1);
        break;
    case 2: {  // a permutation of a contiguous layout
        int64_t nb[4];
        nb[0] = size;
        for (int i = 1; i < 4; ++i) nb[i] = nb[i - 1] * (t.ne[i - 1] > 0 ? t.ne[i - 1] : 1);
        for (int i = 3; i > 0; --i) std::swap(nb[i], nb[rng() % (i + 1)]);
        for (int i = 0; i < 4; ++i) t.nb[i] = nb[i];
        break;
    }
    default:  // anything
        for (int i = 0; i < 4; ++i) t.nb[i] = pick({0, 1, 2, 4, 8, 6, 64, 1280, -4, 1 << 20});
    }
    t.data = rng() % 8 == 0 ? nullptr : arena.data() + (rng() % 256) * 16 + (rng() % 4 == 0 ? rng() % 16 : 0);
    return t;
}

// A tensor shaped for operation `op` half of the time, so that the predicates
// get past their first tests too.
sdhip_tensor like(const sdhip_tensor &base) {
    sdhip_tensor t = tensor();
    if (rng() % 2) {
        for (int i = 0; i < 4; ++i) t.ne[i] = base.ne[i];
        t.type = base.type;
        t.nb[0] = t.type == 1 ? 2 : 4;
        for (int i = 1; i < 4; ++i) t.nb[i] = t.nb[i - 1] * (t.ne[i - 1] > 0 ? t.ne[i - 1] : 1);
    }
    return t;
}

void params(int32_t *p, int n) {
    for (int i = 0; i < n; ++i) p[i] = static_cast<int32_t>(pick({0, 1, 1, 2, 3, -1, 7, 1 << 20}));
}

void operations() {
    const sdhip_tensor a = tensor(), b = like(a), c = like(a), d = like(b);
    sdhip_mul_mat_supported(&a, &b, &c);
    sdhip_mul_mat_work_size(&a, &b, &c);
    sdhip_mul_mat_gated_supported(&a, &b, &c, &d);
    int32_t p[6];
    params(p, 6);
    sdhip_conv2d_supported(&a, &b, &c, p);
    sdhip_conv2d_path(&a, &b, &c, p);
    sdhip_conv2d_work_size(&a, &b, &c, p);
    const float bias = static_cast<float>(pick({0, 0, 1})), cap = static_cast<float>(pick({0, 0, 2}));
    sdhip_attention_supported(&a, &b, &c, &d, bias, cap);
    sdhip_attention_work_size(&a, &b, &c, &d);
    const int groups = static_cast<int>(pick({0, 1, 3, 7, 32, -1, 1 << 20}));
    sdhip_group_norm_supported(&a, &b, groups);
    sdhip_group_norm_work_size(&a, &b, groups);
    sdhip_norm_supported(&a, &b);
    sdhip_token_downsampling(pick({0, 1, 32, 64, 96, -5}), pick({0, 1, 32, 64, 96, 1LL << 40}));
}

// Sources each operation of a ggml graph has.
int sources_of(int op) {
    switch (op) {
    case SDHIP_OP_ADD:
    case SDHIP_OP_MUL:
    case SDHIP_OP_MUL_MAT:
    case SDHIP_OP_CONV_2D:
        return 2;
    case SDHIP_OP_FLASH_ATTN_EXT:
        return 3;
    case SDHIP_OP_NONE:
        return 0;
    case SDHIP_OP_OTHER:
        return static_cast<int>(rng() % 3);
    default:
        return 1;
    }
}

void graph() {
    const int n = 1 + static_cast<int>(rng() % 24);
    std::vector<sdhip_node> leaves(4), nodes(static_cast<size_t>(n));
    for (auto &l : leaves) {
        l = sdhip_node{};
        l.op = SDHIP_OP_NONE;
        l.tensor = tensor();
    }
    std::vector<const sdhip_node *> order;
    for (int i = 0; i < n; ++i) {
        sdhip_node &node = nodes[static_cast<size_t>(i)];
        node = sdhip_node{};
        node.op = static_cast<int32_t>(rng() % (SDHIP_OP_OTHER + 1));
        node.unary = static_cast<int32_t>(rng() % 3);
        node.flags = static_cast<int32_t>(rng() % 4);
        params(node.op_params, SDHIP_MAX_OP_PARAMS);
        node.tensor = tensor();
        const auto source = [&]() -> const sdhip_node * {
            if (i > 0 && rng() % 3) return &nodes[rng() % static_cast<size_t>(i)];
            return &leaves[rng() % leaves.size()];
        };
        const int srcs = sources_of(node.op);
        for (int s = 0; s < srcs; ++s) node.src[s] = source();
        if (node.op >= SDHIP_OP_VIEW && node.op <= SDHIP_OP_TRANSPOSE) node.view_src = node.src[0];
        if (node.op != SDHIP_OP_NONE) {
            // Now and then shaped like its first source, as an operation's
            // output in place of it would be.
            if (node.src[0] != nullptr && rng() % 2) node.tensor = like(node.src[0]->tensor);
            if (node.src[0] != nullptr && rng() % 4 == 0) node.tensor.data = node.src[0]->tensor.data;
        }
        order.push_back(&node);
    }
    for (int i = 0; i < n; ++i) {
        sdhip_node_plan plan{};
        sdhip_plan_nodes(order.data(), n, i, &plan);
        size_t size = 0;
        sdhip_node_work_size(order[static_cast<size_t>(i)], &size);
    }
    sdhip_node_plan plan{};
    sdhip_plan_nodes(order.data(), n, n, &plan);   // past the end
    sdhip_plan_nodes(order.data(), n, -1, &plan);  // before the start
}

const char *kNames[] = {"bits", "input_bits", "group", "weight_group", "quantize", "winograd", "fuse",
                        "fuse_residual", "todo", "todo_tokens", "attention_keys", "gemm_stages", "gemm_tiles",
                        "gemm_core", "qgemm_core", "attention_generic", "attention_fp32", "winograd_splits",
                        "no_such_name", "", "bits=", "=8"};

void tuning() {
    std::string text;
    const int parts = static_cast<int>(rng() % 6);
    for (int i = 0; i < parts; ++i) {
        if (i) text += rng() % 8 ? "," : ",,";
        text += kNames[rng() % (sizeof(kNames) / sizeof(kNames[0]))];
        if (rng() % 6) {
            text += "=";
            text += std::to_string(pick({0, 1, 2, 4, 8, 16, 21, 64, -3, 4294967296LL, 99999999999LL}));
            if (rng() % 10 == 0) text += "x";
        }
    }
    if (rng() % 50 == 0) text.assign(static_cast<size_t>(rng() % 5000), static_cast<char>('a' + rng() % 26));
    sdhip_set_tuning(text.c_str());
    sdhip_last_error();
    sdhip_get_tuning(kNames[rng() % (sizeof(kNames) / sizeof(kNames[0]))]);
}

}  // namespace

int main(int argc, char **argv) {
    const long cases = argc > 1 ? std::atol(argv[1]) : 20000;
    if (argc > 2) rng.seed(std::strtoull(argv[2], nullptr, 10));
    for (long i = 0; i < cases; ++i) {
        if (i % 7 == 0) tuning();
        operations();
        if (i % 4 == 0) graph();
    }
    sdhip_set_tuning("");
    std::printf("host_check: %ld cases, no error\n", cases);
    return 0;
}
