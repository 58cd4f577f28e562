// Memset-free HIP graphs. A captured training step records a memset node for every
// hipMemsetAsync made during capture, including the ones libraries issue themselves (torch's
// multi-block reductions clear their semaphores that way). graph_replace_memsets() rewrites each
// such node, before instantiation, into a kernel node that writes the same bytes with vector
// stores and keeps the node's place in the dependency graph; graph_node_counts() reports what a
// graph holds, so tests can assert that no memset node is left.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

namespace dopt {
namespace {

constexpr int FILL_THREADS = 256;
constexpr uint64_t FILL_MAX_BLOCKS = 2048;

// Contiguous fill of nbytes bytes at dst. `pattern` holds the memset value replicated to 32 bits
// (period = element size, which divides 4); dst is element-aligned, so the byte at address a is
// byte a % 4 of the pattern. 16-byte stores in the aligned body, byte stores in head and tail.
__global__ __launch_bounds__(FILL_THREADS) void graph_fill_bytes_kernel(uint8_t* dst, uint64_t nbytes, uint32_t pattern) {
    const uint64_t a0 = (uint64_t)dst;
    uint64_t head = (16 - (a0 & 15)) & 15;
    if (head > nbytes) head = nbytes;
    const uint64_t nvec = (nbytes - head) >> 4;
    const uint64_t tail = head + (nvec << 4);
    const uint64_t tid = (uint64_t)blockIdx.x * FILL_THREADS + threadIdx.x;
    const uint64_t stride = (uint64_t)gridDim.x * FILL_THREADS;
    const uint4 v = make_uint4(pattern, pattern, pattern, pattern);
    uint4* body = (uint4*)(dst + head);
    for (uint64_t i = tid; i < nvec; i += stride) body[i] = v;
    for (uint64_t i = tid; i < head; i += stride) dst[i] = (uint8_t)(pattern >> (8 * ((a0 + i) & 3)));
    for (uint64_t i = tail + tid; i < nbytes; i += stride) dst[i] = (uint8_t)(pattern >> (8 * ((a0 + i) & 3)));
}

// Pitched fill: height rows of width elements of esize (1, 2 or 4) bytes, rows pitch bytes apart.
__global__ __launch_bounds__(FILL_THREADS) void graph_fill_rows_kernel(uint8_t* dst, uint64_t pitch, uint64_t width,
                                                                        uint64_t height, uint32_t value, uint32_t esize) {
    const uint64_t n = width * height;
    const uint64_t stride = (uint64_t)gridDim.x * FILL_THREADS;
    for (uint64_t i = (uint64_t)blockIdx.x * FILL_THREADS + threadIdx.x; i < n; i += stride) {
        const uint64_t r = i / width, c = i - r * width;
        uint8_t* p = dst + r * pitch + c * esize;
        if (esize == 4)
            *(uint32_t*)p = value;
        else if (esize == 2)
            *(uint16_t*)p = (uint16_t)value;
        else
            *p = (uint8_t)value;
    }
}

uint32_t fill_blocks(uint64_t work) {
    const uint64_t b = (work + FILL_THREADS - 1) / FILL_THREADS;
    return (uint32_t)(b < 1 ? 1 : b > FILL_MAX_BLOCKS ? FILL_MAX_BLOCKS : b);
}

bool get_nodes(hipGraph_t g, std::vector<hipGraphNode_t>& out) {
    size_t n = 0;
    if (hipGraphGetNodes(g, nullptr, &n) != hipSuccess) return false;
    out.resize(n);
    return n == 0 || hipGraphGetNodes(g, out.data(), &n) == hipSuccess;
}

bool get_edges(hipGraphNode_t node, std::vector<hipGraphNode_t>& deps, std::vector<hipGraphNode_t>& dependents) {
    size_t nd = 0, nt = 0;
    if (hipGraphNodeGetDependencies(node, nullptr, &nd) != hipSuccess) return false;
    if (hipGraphNodeGetDependentNodes(node, nullptr, &nt) != hipSuccess) return false;
    deps.resize(nd);
    dependents.resize(nt);
    if (nd && hipGraphNodeGetDependencies(node, deps.data(), &nd) != hipSuccess) return false;
    if (nt && hipGraphNodeGetDependentNodes(node, dependents.data(), &nt) != hipSuccess) return false;
    return true;
}

}  // namespace

// Adds the node count of g (child graphs included) per hipGraphNodeType to counts[0..n_counts).
// Returns the name of the failing HIP call, or nullptr.
const char* graph_node_counts(hipGraph_t g, int64_t* counts, int n_counts) {
    std::vector<hipGraphNode_t> nodes;
    if (!get_nodes(g, nodes)) return "hipGraphGetNodes";
    for (hipGraphNode_t node : nodes) {
        hipGraphNodeType t;
        if (hipGraphNodeGetType(node, &t) != hipSuccess) return "hipGraphNodeGetType";
        if ((int)t >= 0 && (int)t < n_counts) ++counts[(int)t];
        if (t == hipGraphNodeTypeGraph) {
            hipGraph_t child;
            if (hipGraphChildGraphNodeGetGraph(node, &child) != hipSuccess) return "hipGraphChildGraphNodeGetGraph";
            if (const char* e = graph_node_counts(child, counts, n_counts)) return e;
        }
    }
    return nullptr;
}

// Replaces every memset node of g (child graphs included) by a fill kernel node with the same
// dependencies and dependents; adds the number replaced to *replaced. Returns the name of the
// failing HIP call, or nullptr.
const char* graph_replace_memsets(hipGraph_t g, int64_t* replaced) {
    std::vector<hipGraphNode_t> nodes, deps, dependents;
    if (!get_nodes(g, nodes)) return "hipGraphGetNodes";
    for (hipGraphNode_t node : nodes) {
        hipGraphNodeType t;
        if (hipGraphNodeGetType(node, &t) != hipSuccess) return "hipGraphNodeGetType";
        if (t == hipGraphNodeTypeGraph) {
            hipGraph_t child;
            if (hipGraphChildGraphNodeGetGraph(node, &child) != hipSuccess) return "hipGraphChildGraphNodeGetGraph";
            if (const char* e = graph_replace_memsets(child, replaced)) return e;
            continue;
        }
        if (t != hipGraphNodeTypeMemset) continue;
        hipMemsetParams p{};
        if (hipGraphMemsetNodeGetParams(node, &p) != hipSuccess) return "hipGraphMemsetNodeGetParams";
        const uint32_t es = p.elementSize;
        if (es != 1 && es != 2 && es != 4) return "memset node element size";
        uint8_t* dst = (uint8_t*)p.dst;
        uint64_t pitch = p.pitch, width = p.width, height = p.height ? p.height : 1;
        uint64_t nbytes = width * es * height;
        uint32_t value = p.value, esize = es;
        uint32_t pattern = es == 1 ? (value & 0xffu) * 0x01010101u : es == 2 ? (value & 0xffffu) * 0x00010001u : value;
        void* args_bytes[3] = {&dst, &nbytes, &pattern};
        void* args_rows[6] = {&dst, &pitch, &width, &height, &value, &esize};
        hipKernelNodeParams kp{};
        kp.blockDim = dim3(FILL_THREADS);
        kp.sharedMemBytes = 0;
        kp.extra = nullptr;
        if (height == 1 || pitch == width * es) {
            kp.func = (void*)graph_fill_bytes_kernel;
            kp.gridDim = dim3(fill_blocks((nbytes + 15) / 16));
            kp.kernelParams = args_bytes;
        } else {
            kp.func = (void*)graph_fill_rows_kernel;
            kp.gridDim = dim3(fill_blocks(width * height));
            kp.kernelParams = args_rows;
        }
        if (!get_edges(node, deps, dependents)) return "hipGraphNodeGetDependencies";
        hipGraphNode_t k;
        if (hipGraphAddKernelNode(&k, g, deps.empty() ? nullptr : deps.data(), deps.size(), &kp) != hipSuccess)
            return "hipGraphAddKernelNode";
        for (hipGraphNode_t d : dependents)
            if (hipGraphAddDependencies(g, &k, &d, 1) != hipSuccess) return "hipGraphAddDependencies";
        if (hipGraphDestroyNode(node) != hipSuccess) return "hipGraphDestroyNode";
        ++*replaced;
    }
    return nullptr;
}

}  // namespace dopt
