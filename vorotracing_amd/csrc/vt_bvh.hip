// vt_bvh.hip -- start-cell lookup: a linear BVH over the sites (replaces the
// cuBQL BinaryBVH of nn_bvh.cu:12-117) and an exact nearest-site query.
//
// Build: bounding box -> 30-bit Morton codes -> stable radix sort -> binary
// radix tree over the sorted codes (Karras 2012, ties in the code broken by
// sorted position) -> bottom-up refit.  Each internal node stores both
// children's boxes, so a query tests two boxes per node fetch.
// Query: depth-first, nearer child first, exact: squared distance
// dot(q - p, q - p) (fma convention) and ties to the lowest site index, with
// conservative box pruning so rounding can never drop a closer site.
#include "vt_internal.h"
#include "vt_prims.h"
#include "vt_device.h"

#include <mutex>

namespace vt {

struct BvhNode {          // 64 bytes
    float lo[2][3];       // child boxes: [0] = left, [1] = right
    float hi[2][3];
    uint32_t child[2];    // LEAF bit | sorted leaf position, or internal index
    uint32_t parent, pad; // parent internal index (NONE for the root)
};

constexpr uint32_t LEAF = 0x80000000u;

struct BvhHandle {
    uint32_t n = 0, cap = 0;
    BvhNode *nodes = nullptr;    // n-1 internal nodes
    uint32_t *leaf_idx = nullptr; // sorted position -> site index
    uint32_t *leaf_parent = nullptr;
    uint32_t *flags = nullptr;
    uint32_t *ws = nullptr;
    size_t ws_words = 0;
    float *bb = nullptr;
    uint32_t stack_limit = 64; // traversal stack entries a query may use (test hook)
    bool force_tree = false;   // queries always walk the tree (test hook)
};

__device__ __forceinline__ int bvh_delta(const uint32_t *__restrict__ keys, uint32_t n, int i, int j)
{
    if (j < 0 || j >= (int)n)
        return -1;
    uint32_t a = keys[i], b = keys[j];
    if (a != b)
        return __builtin_clz(a ^ b);
    return 32 + __builtin_clz((uint32_t)i ^ (uint32_t)j);
}

__global__ void bvh_keys_kernel(const float *__restrict__ points, uint32_t n, const float *__restrict__ bb,
                                uint32_t *__restrict__ keys, uint32_t *__restrict__ vals)
{
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n)
        return;
    f3 p = load_site(points, i);
    float v[3] = {p.x, p.y, p.z};
    uint32_t q[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        float size = __builtin_fmaxf(bb[3 + c] - bb[c], 1e-30f);
        float x = ((v[c] - bb[c]) / size) * 1023.0f;
        q[c] = (uint32_t)__builtin_fminf(__builtin_fmaxf(x, 0.0f), 1023.0f);
    }
    uint32_t code = 0;
#pragma unroll
    for (int b = 0; b < 10; ++b)
        code |= (((q[0] >> b) & 1u) << (3 * b + 2)) | (((q[1] >> b) & 1u) << (3 * b + 1)) |
                (((q[2] >> b) & 1u) << (3 * b));
    keys[i] = code;
    vals[i] = i;
}

// Karras 2012, internal node i of n-1
__global__ void bvh_hierarchy_kernel(const uint32_t *__restrict__ keys, uint32_t n, BvhNode *__restrict__ nodes,
                                     uint32_t *__restrict__ leaf_parent, uint32_t *__restrict__ flags)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int)n - 1)
        return;
    flags[i] = 0;
    int d = (bvh_delta(keys, n, i, i + 1) - bvh_delta(keys, n, i, i - 1)) >= 0 ? 1 : -1;
    int dmin = bvh_delta(keys, n, i, i - d);
    int lmax = 2;
    while (bvh_delta(keys, n, i, i + lmax * d) > dmin)
        lmax *= 2;
    int l = 0;
    for (int t = lmax / 2; t >= 1; t /= 2)
        if (bvh_delta(keys, n, i, i + (l + t) * d) > dmin)
            l += t;
    int j = i + l * d;
    int dnode = bvh_delta(keys, n, i, j);
    int s = 0;
    int div = 2;
    int t = (l + div - 1) / div;
    for (;;) {
        if (bvh_delta(keys, n, i, i + (s + t) * d) > dnode)
            s += t;
        if (t == 1)
            break;
        div *= 2;
        t = (l + div - 1) / div;
    }
    int gamma = i + s * d + min(d, 0);
    int lo = min(i, j), hi = max(i, j);
    uint32_t left = (lo == gamma) ? (LEAF | (uint32_t)gamma) : (uint32_t)gamma;
    uint32_t right = (hi == gamma + 1) ? (LEAF | (uint32_t)(gamma + 1)) : (uint32_t)(gamma + 1);
    nodes[i].child[0] = left;
    nodes[i].child[1] = right;
    if (left & LEAF)
        leaf_parent[left & ~LEAF] = (uint32_t)i;
    else
        nodes[left].parent = (uint32_t)i;
    if (right & LEAF)
        leaf_parent[right & ~LEAF] = (uint32_t)i;
    else
        nodes[right].parent = (uint32_t)i;
    if (i == 0)
        nodes[0].parent = NONE;
}

// Bottom-up refit, one launch per tree level and no memory fences: a node
// enters a level's list when the second of its two children has written its
// box into the node's child slot (an atomic count per node), and the next
// launch reads both boxes, which the kernel boundary has made visible on
// every XCD.  A node's box goes into its parent's slot, and so on up to the
// root.  The split prefix lengthens strictly from a node to its children
// (delta 2..31 for distinct 30-bit codes, 33..63 for index ties), so no path
// has more than 61 internal nodes; BVH_LEVELS launches cover every tree.
constexpr int BVH_LEVELS = 64;

__device__ __forceinline__ void put_child_box(BvhNode *nodes, uint32_t parent, uint32_t child, const float *lo,
                                              const float *hi)
{
    const int side = nodes[parent].child[0] == child ? 0 : 1;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        nodes[parent].lo[side][c] = lo[c];
        nodes[parent].hi[side][c] = hi[c];
    }
}

// the second child to arrive appends `node` to a level list
__device__ __forceinline__ void arrive(uint32_t *flags, uint32_t node, uint32_t *list, uint32_t *count)
{
    if (atomicAdd(&flags[node], 1u) == 1u)
        list[atomicAdd(count, 1u)] = node;
}

__global__ void bvh_leaf_boxes_kernel(const float *__restrict__ points, const uint32_t *__restrict__ leaf_idx,
                                      uint32_t n, BvhNode *nodes, const uint32_t *__restrict__ leaf_parent,
                                      uint32_t *flags, uint32_t *list0, uint32_t *counters)
{
    const uint32_t k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= n)
        return;
    const f3 p = load_site(points, leaf_idx[k]);
    const float b[3] = {p.x, p.y, p.z};
    const uint32_t parent = leaf_parent[k];
    put_child_box(nodes, parent, LEAF | k, b, b);
    arrive(flags, parent, list0, &counters[0]);
}

// nodes of `in` (counters[level] of them): box = union of the two child
// boxes, written into the parent's slot
__global__ void bvh_level_kernel(BvhNode *nodes, uint32_t *flags, const uint32_t *__restrict__ in, uint32_t *out,
                                 uint32_t *counters, int level)
{
    const uint32_t cnt = counters[level];
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < cnt; i += gridDim.x * blockDim.x) {
        const uint32_t node = in[i];
        const BvhNode nd = nodes[node];
        if (nd.parent == NONE)
            continue;
        float lo[3], hi[3];
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            lo[c] = __builtin_fminf(nd.lo[0][c], nd.lo[1][c]);
            hi[c] = __builtin_fmaxf(nd.hi[0][c], nd.hi[1][c]);
        }
        put_child_box(nodes, nd.parent, node, lo, hi);
        arrive(flags, nd.parent, out, &counters[level + 1]);
    }
}

__global__ void bvh_zero_kernel(uint32_t *p, uint32_t n)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        p[i] = 0u;
}

__device__ __forceinline__ float box_d2(f3 q, const float *lo, const float *hi)
{
    float dx = __builtin_fmaxf(__builtin_fmaxf(lo[0] - q.x, 0.0f), q.x - hi[0]);
    float dy = __builtin_fmaxf(__builtin_fmaxf(lo[1] - q.y, 0.0f), q.y - hi[1]);
    float dz = __builtin_fmaxf(__builtin_fmaxf(lo[2] - q.z, 0.0f), q.z - hi[2]);
    return fma_(dz, dz, fma_(dy, dy, dx * dx));
}

// prune a box only when its distance exceeds the best by more than the
// rounding of either computation (relative 2^-16 margin)
__device__ __forceinline__ bool box_may_hold(float bd2, float best) { return bd2 * 0.9999847f <= best; }

constexpr int BVH_STACK = 64;

// Nearest site of q: the smallest squared distance, the lowest site index
// among equal distances.
__device__ __forceinline__ uint32_t bvh_nearest(f3 q, const BvhNode *__restrict__ nodes,
                                                const uint32_t *__restrict__ leaf_idx, uint32_t n,
                                                const float *__restrict__ points, uint32_t stack_limit)
{
    float best = __builtin_huge_valf();
    uint32_t best_i = NONE;
    auto visit_leaf = [&](uint32_t k) {
        uint32_t idx = leaf_idx[k];
        f3 df = sub(q, load_site(points, idx));
        float d2 = dot(df, df);
        if (d2 < best || (d2 == best && idx < best_i)) {
            best = d2;
            best_i = idx;
        }
    };
    bool overflow = false;
    if (n == 1) {
        visit_leaf(0);
    } else {
        uint32_t stack[BVH_STACK];
        float sdist[BVH_STACK];
        int sp = 0;
        stack[sp] = 0;
        sdist[sp] = 0.0f;
        sp++;
        while (sp > 0) {
            sp--;
            uint32_t node = stack[sp];
            if (!box_may_hold(sdist[sp], best))
                continue;
            const BvhNode &nd = nodes[node];
            float d0 = box_d2(q, nd.lo[0], nd.hi[0]);
            float d1 = box_d2(q, nd.lo[1], nd.hi[1]);
            uint32_t c0 = nd.child[0], c1 = nd.child[1];
            // visit / push the farther child first so the nearer is expanded next
            if (d1 < d0) {
                uint32_t tc = c0;
                c0 = c1;
                c1 = tc;
                float td = d0;
                d0 = d1;
                d1 = td;
            }
            if (box_may_hold(d1, best)) {
                if (c1 & LEAF)
                    visit_leaf(c1 & ~LEAF);
                else if (sp < (int)stack_limit) {
                    stack[sp] = c1;
                    sdist[sp] = d1;
                    sp++;
                } else {
                    overflow = true;
                }
            }
            if (box_may_hold(d0, best)) {
                if (c0 & LEAF)
                    visit_leaf(c0 & ~LEAF);
                else if (sp < (int)stack_limit) {
                    stack[sp] = c0;
                    sdist[sp] = d0;
                    sp++;
                } else {
                    overflow = true;
                }
            }
        }
    }
    if (overflow) {
        // A subtree was not searched (stack full: cannot happen while the
        // tree is at most 30 + 31 levels deep, i.e. n < 2^31, but a wrong
        // start cell must never be returned): answer by a scan of all sites,
        // with the same distance and tie rule.
        best = __builtin_huge_valf();
        best_i = NONE;
        for (uint32_t k = 0; k < n; ++k) {
            const f3 df = sub(q, load_site(points, k));
            const float d2 = dot(df, df);
            if (d2 < best) { // k increases, so ties keep the lowest index
                best = d2;
                best_i = k;
            }
        }
    }
    return best_i;
}

__global__ __launch_bounds__(256) void bvh_query_kernel(const BvhNode *__restrict__ nodes,
                                                        const uint32_t *__restrict__ leaf_idx, uint32_t n,
                                                        const float *__restrict__ points,
                                                        const float *__restrict__ queries, uint32_t nq,
                                                        int32_t *__restrict__ out, uint32_t stack_limit)
{
    uint32_t qi = xcd_block_linear();
    if (qi >= nq)
        return;
    out[qi] = (int32_t)bvh_nearest(load_site(queries, qi), nodes, leaf_idx, n, points, stack_limit);
}

// ---- start cells of a ray batch --------------------------------------------
//
// The nearest site of every ray's origin, one tree query per run of equal
// consecutive origins (the rays of a camera share one origin, or one per
// row under a rolling shutter), without the host learning the number of
// runs: flags, a scan, the runs' origins compacted, a grid-stride query over
// the device-side run count, and a gather.

constexpr uint32_t RUN_QUERY_BLOCKS = 2048;

__device__ __forceinline__ f3 ray_origin(const float *__restrict__ rays, uint32_t i)
{
    return mk(rays[6 * (size_t)i], rays[6 * (size_t)i + 1], rays[6 * (size_t)i + 2]);
}

// flags[i] = 1 where ray i starts a run (its origin differs from ray i-1's)
__global__ void run_flags_kernel(const float *__restrict__ rays, uint32_t num_rays, uint32_t *__restrict__ flags)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= num_rays)
        return;
    bool start = i == 0;
    if (!start) {
        const f3 a = ray_origin(rays, i), b = ray_origin(rays, i - 1);
        start = a.x != b.x || a.y != b.y || a.z != b.z;
    }
    flags[i] = start ? 1u : 0u;
}

// runs' origins packed in run order; count = the number of runs
__global__ void run_compact_kernel(const float *__restrict__ rays, const uint32_t *__restrict__ flags,
                                   const uint32_t *__restrict__ first, uint32_t num_rays, float *__restrict__ origins,
                                   uint32_t *__restrict__ count)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= num_rays)
        return;
    if (flags[i]) {
        const f3 o = ray_origin(rays, i);
        origins[3 * (size_t)first[i]] = o.x;
        origins[3 * (size_t)first[i] + 1] = o.y;
        origins[3 * (size_t)first[i] + 2] = o.z;
    }
    if (i == num_rays - 1)
        *count = first[i] + flags[i];
}

__global__ __launch_bounds__(256) void run_query_kernel(const BvhNode *__restrict__ nodes,
                                                        const uint32_t *__restrict__ leaf_idx, uint32_t n,
                                                        const float *__restrict__ points,
                                                        const float *__restrict__ origins,
                                                        const uint32_t *__restrict__ count,
                                                        uint32_t *__restrict__ nearest, uint32_t stack_limit)
{
    const uint32_t runs = *count;
    for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < runs; j += gridDim.x * blockDim.x)
        nearest[j] = bvh_nearest(load_site(origins, j), nodes, leaf_idx, n, points, stack_limit);
}

// start[i] = the nearest site of ray i's run
__global__ void run_gather_kernel(const uint32_t *__restrict__ flags, const uint32_t *__restrict__ first,
                                  uint32_t num_rays, const uint32_t *__restrict__ nearest, uint32_t *__restrict__ start)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < num_rays)
        start[i] = nearest[first[i] + flags[i] - 1u];
}

// Few queries (num_queries * num_points <= NN_SCAN_PAIRS and at most
// NN_SCAN_MAX_QUERIES, e.g. the one camera origin of a pinhole frame): the
// tree walk is a chain of dependent loads on one lane (about 37 us for 1M
// sites), while a scan of all sites by the whole GPU reads 12 bytes per site
// once.  Same squared distance and the same lowest-index rule as the tree, so
// the answer is the same site.  The scan launches NN_SCAN_BLOCKS blocks per
// query whatever the site count, so many queries over few sites walk the tree
// (each then costs one lane, not 1024 blocks and 8 KiB of partials).
constexpr uint64_t NN_SCAN_PAIRS = 1ull << 26;
constexpr uint32_t NN_SCAN_MAX_QUERIES = 64;
constexpr int NN_SCAN_BLOCK = 256;
constexpr uint32_t NN_SCAN_BLOCKS = 1024; // per query
constexpr uint32_t NN_SCAN_UNROLL = 4;    // sites per lane and pass of nn_scan_kernel

__device__ __forceinline__ bool nn_better(float d, uint32_t i, float bd, uint32_t bi)
{
    return d < bd || (d == bd && i < bi);
}

// partial[q * NN_SCAN_BLOCKS + block] = (squared distance bits, site) of the
// nearest site among the sites this block strides over; grid (blocks, queries)
__global__ __launch_bounds__(NN_SCAN_BLOCK) void nn_scan_kernel(const float *__restrict__ points, uint32_t n,
                                                                const float *__restrict__ queries,
                                                                uint2 *__restrict__ partial)
{
    __shared__ float sd[NN_SCAN_BLOCK / 64];
    __shared__ uint32_t si[NN_SCAN_BLOCK / 64];
    const uint32_t qi = blockIdx.y;
    const f3 q = load_site(queries, qi);
    float best = __builtin_huge_valf();
    uint32_t bi = NONE;
    // NN_SCAN_UNROLL sites per pass, their loads issued together
    constexpr uint32_t stride = NN_SCAN_BLOCKS * NN_SCAN_BLOCK;
    for (uint32_t i0 = blockIdx.x * NN_SCAN_BLOCK + threadIdx.x; i0 < n; i0 += NN_SCAN_UNROLL * stride) {
        f3 site[NN_SCAN_UNROLL];
#pragma unroll
        for (uint32_t u = 0; u < NN_SCAN_UNROLL; ++u) {
            const uint32_t i = i0 + u * stride;
            site[u] = load_site(points, i < n ? i : i0);
        }
#pragma unroll
        for (uint32_t u = 0; u < NN_SCAN_UNROLL; ++u) {
            const uint32_t i = i0 + u * stride;
            const f3 df = sub(q, site[u]);
            const float d2 = dot(df, df);
            if (i < n && d2 < best) { // i increases along the stride, so ties keep the lower index
                best = d2;
                bi = i;
            }
        }
    }
    for (int o = 32; o >= 1; o >>= 1) {
        const float od = __shfl_xor(best, o, 64);
        const uint32_t oi = __shfl_xor(bi, o, 64);
        if (nn_better(od, oi, best, bi)) {
            best = od;
            bi = oi;
        }
    }
    const uint32_t wv = threadIdx.x >> 6;
    if ((threadIdx.x & 63u) == 0) {
        sd[wv] = best;
        si[wv] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t k = 1; k < NN_SCAN_BLOCK / 64; ++k)
            if (nn_better(sd[k], si[k], best, bi)) {
                best = sd[k];
                bi = si[k];
            }
        partial[(size_t)qi * NN_SCAN_BLOCKS + blockIdx.x] = make_uint2(f_bits(best), bi);
    }
}

// out[q] = the best of the query's NN_SCAN_BLOCKS partials; one wave per query
__global__ __launch_bounds__(64) void nn_pick_kernel(const uint2 *__restrict__ partial, int32_t *__restrict__ out)
{
    const uint32_t qi = blockIdx.x;
    float best = __builtin_huge_valf();
    uint32_t bi = NONE;
    // the partials' loads issued together (a loop of dependent round trips took 7 us)
    static_assert(NN_SCAN_BLOCKS % 64 == 0, "partials per lane");
#pragma unroll
    for (uint32_t j = 0; j < NN_SCAN_BLOCKS / 64; ++j) {
        const uint2 p = partial[(size_t)qi * NN_SCAN_BLOCKS + threadIdx.x + 64 * j];
        if (nn_better(bits_f(p.x), p.y, best, bi)) {
            best = bits_f(p.x);
            bi = p.y;
        }
    }
    for (int o = 32; o >= 1; o >>= 1) {
        const float od = __shfl_xor(best, o, 64);
        const uint32_t oi = __shfl_xor(bi, o, 64);
        if (nn_better(od, oi, best, bi)) {
            best = od;
            bi = oi;
        }
    }
    if (threadIdx.x == 0)
        out[qi] = (int32_t)bi;
}

static int ensure_capacity(BvhHandle *h, uint32_t n)
{
    if (n <= h->cap && h->nodes)
        return VT_OK;
    hipFree(h->nodes);
    hipFree(h->leaf_idx);
    hipFree(h->leaf_parent);
    hipFree(h->flags);
    hipFree(h->ws);
    hipFree(h->bb);
    h->nodes = nullptr;
    h->leaf_idx = h->leaf_parent = h->flags = h->ws = nullptr;
    h->bb = nullptr;
    h->cap = 0;
    size_t ws_words = 2 * (size_t)n + radix_sort_workspace_words(n) + 16;
    VT_HIP_CHECK(hipMalloc(&h->nodes, sizeof(BvhNode) * (size_t)(n > 1 ? n - 1 : 1)));
    VT_HIP_CHECK(hipMalloc(&h->leaf_idx, 4 * (size_t)n));
    VT_HIP_CHECK(hipMalloc(&h->leaf_parent, 4 * (size_t)n));
    VT_HIP_CHECK(hipMalloc(&h->flags, 4 * (size_t)(n > 1 ? n - 1 : 1)));
    VT_HIP_CHECK(hipMalloc(&h->ws, 4 * ws_words));
    VT_HIP_CHECK(hipMalloc(&h->bb, 8 * sizeof(float)));
    h->ws_words = ws_words;
    h->cap = n;
    return VT_OK;
}

} // namespace vt

using namespace vt;

extern "C" int vt_bvh_create(void **handle)
{
    clear_error();
    VT_REQUIRE(handle, "null handle pointer");
    *handle = new BvhHandle();
    return VT_OK;
}

extern "C" int vt_bvh_destroy(void *handle)
{
    clear_error();
    BvhHandle *h = (BvhHandle *)handle;
    if (!h)
        return VT_OK;
    hipFree(h->nodes);
    hipFree(h->leaf_idx);
    hipFree(h->leaf_parent);
    hipFree(h->flags);
    hipFree(h->ws);
    hipFree(h->bb);
    delete h;
    return VT_OK;
}

extern "C" int vt_bvh_build(void *handle, const float *points, uint32_t num_points, vt_stream_t stream)
{
    clear_error();
    BvhHandle *h = (BvhHandle *)handle;
    VT_REQUIRE(h, "null BVH handle");
    VT_REQUIRE(points || num_points == 0, "null points");
    VT_REQUIRE(num_points < 0x7fffffffu, "too many points");
    hipStream_t s = as_stream(stream);
    h->n = 0;
    if (num_points == 0)
        return VT_OK;
    int rc = ensure_capacity(h, num_points);
    if (rc)
        return rc;
    uint32_t n = num_points;
    uint32_t *keys = h->ws;
    uint32_t *sws = h->ws + n;
    uint32_t *bbw = sws + radix_sort_workspace_words(n);
    rc = bbox3(points, n, h->bb, bbw, s);
    if (rc)
        return rc;
    bvh_keys_kernel<<<(n + 255) / 256, 256, 0, s>>>(points, n, h->bb, keys, h->leaf_idx);
    VT_LAUNCH_CHECK("bvh_keys_kernel");
    rc = radix_sort_pairs(keys, h->leaf_idx, n, 30, sws, s);
    if (rc)
        return rc;
    if (n > 1) {
        bvh_hierarchy_kernel<<<(n - 1 + 255) / 256, 256, 0, s>>>(keys, n, h->nodes, h->leaf_parent, h->flags);
        VT_LAUNCH_CHECK("bvh_hierarchy_kernel");
        // level lists (n words each) and BVH_LEVELS + 1 counters in the sort
        // workspace, free once the tree is built (ws_words >= 4n + 272)
        uint32_t *lists[2] = {h->ws, h->ws + n};
        uint32_t *counters = h->ws + 2 * (size_t)n;
        bvh_zero_kernel<<<1, 128, 0, s>>>(counters, BVH_LEVELS + 1);
        VT_LAUNCH_CHECK("bvh_zero_kernel");
        bvh_leaf_boxes_kernel<<<(n + 255) / 256, 256, 0, s>>>(points, h->leaf_idx, n, h->nodes, h->leaf_parent,
                                                              h->flags, lists[0], counters);
        VT_LAUNCH_CHECK("bvh_leaf_boxes_kernel");
        const uint32_t blocks = (uint32_t)(((size_t)n / 2 + 255) / 256 < 1024 ? ((size_t)n / 2 + 255) / 256 : 1024);
        for (int level = 0; level < BVH_LEVELS; ++level) {
            bvh_level_kernel<<<blocks ? blocks : 1, 256, 0, s>>>(h->nodes, h->flags, lists[level & 1],
                                                                lists[(level + 1) & 1], counters, level);
            VT_LAUNCH_CHECK("bvh_level_kernel");
        }
    }
    h->n = n;
    return VT_OK;
}

namespace vt {

// The all-sites scan (nn_scan_kernel + nn_pick_kernel) into `partial`
// (num_queries * NN_SCAN_BLOCKS entries).
static int launch_scan(const float *points, uint32_t num_points, const float *queries, uint32_t num_queries,
                       uint2 *partial, int32_t *out, hipStream_t stream)
{
    nn_scan_kernel<<<dim3(NN_SCAN_BLOCKS, num_queries), NN_SCAN_BLOCK, 0, stream>>>(points, num_points, queries,
                                                                                   partial);
    VT_LAUNCH_CHECK("nn_scan_kernel");
    nn_pick_kernel<<<num_queries, 64, 0, stream>>>(partial, out);
    VT_LAUNCH_CHECK("nn_pick_kernel");
    return VT_OK;
}

static bool scan_is_faster(const BvhHandle *h, uint32_t num_queries)
{
    return !h->force_tree && (uint64_t)num_queries * h->n <= NN_SCAN_PAIRS && num_queries <= NN_SCAN_MAX_QUERIES;
}

static int query_common(BvhHandle *h, const float *points, uint32_t num_points, const float *queries,
                        uint32_t num_queries, int32_t *out, uint2 *partial, size_t partial_entries,
                        hipStream_t stream)
{
    VT_REQUIRE(h, "null BVH handle");
    VT_REQUIRE(h->n > 0, "BVH must be built before querying");
    VT_REQUIRE(num_points == h->n, "points must be the point set the BVH was built on (%u vs %u)", num_points, h->n);
    if (num_queries == 0)
        return VT_OK;
    VT_REQUIRE(points && queries && out, "null pointer argument");
    if (partial && scan_is_faster(h, num_queries) && (size_t)num_queries * NN_SCAN_BLOCKS <= partial_entries)
        return launch_scan(points, h->n, queries, num_queries, partial, out, stream);
    bvh_query_kernel<<<(num_queries + 255) / 256, 256, 0, stream>>>(
        h->nodes, h->leaf_idx, h->n, points, queries, num_queries, out,
        h->stack_limit < (uint32_t)BVH_STACK ? h->stack_limit : (uint32_t)BVH_STACK);
    VT_LAUNCH_CHECK("bvh_query_kernel");
    return VT_OK;
}

} // namespace vt

extern "C" int vt_bvh_query(void *handle, const float *points, uint32_t num_points, const float *queries,
                            uint32_t num_queries, int32_t *out, vt_stream_t stream)
{
    clear_error();
    BvhHandle *h = (BvhHandle *)handle;
    // the scan's partials live in the handle's workspace when it has room
    return query_common(h, points, num_points, queries, num_queries, out,
                        h ? reinterpret_cast<uint2 *>(h->ws) : nullptr, h ? h->ws_words / 2 : 0, as_stream(stream));
}

extern "C" size_t vt_nearest_scan_workspace_size(uint32_t num_queries)
{
    return (size_t)num_queries * NN_SCAN_BLOCKS * sizeof(uint2);
}

extern "C" int vt_bvh_query_ws(void *handle, const float *points, uint32_t num_points, const float *queries,
                               uint32_t num_queries, int32_t *out, void *workspace, size_t workspace_bytes,
                               vt_stream_t stream)
{
    clear_error();
    VT_REQUIRE(!workspace_bytes || workspace, "null workspace with a nonzero size");
    VT_REQUIRE(((uintptr_t)workspace & 7u) == 0, "workspace must be 8-byte aligned");
    return query_common((BvhHandle *)handle, points, num_points, queries, num_queries, out,
                        reinterpret_cast<uint2 *>(workspace), workspace_bytes / sizeof(uint2), as_stream(stream));
}

// workspace (u32 words): flags, first ray of each run (num_rays each), the
// runs' origins (3 num_rays floats), their nearest sites (num_rays), the run
// count, then the scan's workspace
extern "C" size_t vt_start_cells_workspace_size(uint32_t num_rays)
{
    return (6 * (size_t)num_rays + 1 + scan_workspace_words(num_rays)) * 4;
}

extern "C" int vt_start_cells(void *handle, const float *points, uint32_t num_points, const float *rays,
                              uint32_t num_rays, uint32_t *start, void *workspace, vt_stream_t stream)
{
    clear_error();
    BvhHandle *h = (BvhHandle *)handle;
    VT_REQUIRE(h, "null BVH handle");
    VT_REQUIRE(h->n > 0, "BVH must be built before querying");
    VT_REQUIRE(num_points == h->n, "points must be the point set the BVH was built on (%u vs %u)", num_points, h->n);
    if (num_rays == 0)
        return VT_OK;
    VT_REQUIRE(points && rays && start && workspace, "null pointer argument");
    VT_REQUIRE(((uintptr_t)workspace & 3u) == 0, "workspace must be 4-byte aligned");
    hipStream_t s = as_stream(stream);
    uint32_t *flags = static_cast<uint32_t *>(workspace);
    uint32_t *first = flags + num_rays;
    float *origins = reinterpret_cast<float *>(first + num_rays);
    uint32_t *nearest = reinterpret_cast<uint32_t *>(origins + 3 * (size_t)num_rays);
    uint32_t *count = nearest + num_rays;
    uint32_t *sws = count + 1;
    const uint32_t blocks = (num_rays + 255) / 256;
    run_flags_kernel<<<blocks, 256, 0, s>>>(rays, num_rays, flags);
    VT_LAUNCH_CHECK("run_flags_kernel");
    int rc = exclusive_scan_u32(flags, first, num_rays, sws, s);
    if (rc)
        return rc;
    run_compact_kernel<<<blocks, 256, 0, s>>>(rays, flags, first, num_rays, origins, count);
    VT_LAUNCH_CHECK("run_compact_kernel");
    run_query_kernel<<<blocks < RUN_QUERY_BLOCKS ? blocks : RUN_QUERY_BLOCKS, 256, 0, s>>>(
        h->nodes, h->leaf_idx, h->n, points, origins, count, nearest,
        h->stack_limit < (uint32_t)BVH_STACK ? h->stack_limit : (uint32_t)BVH_STACK);
    VT_LAUNCH_CHECK("run_query_kernel");
    run_gather_kernel<<<blocks, 256, 0, s>>>(flags, first, num_rays, nearest, start);
    VT_LAUNCH_CHECK("run_gather_kernel");
    return VT_OK;
}

// ---- allocation-free nearest-site scan -------------------------------------
//
// The few-query path of vt_bvh_query (nn_scan_kernel + nn_pick_kernel) with
// its per-block partials in a file-scope device array instead of a handle's
// hipMalloc'd workspace, for callers that cannot allocate (code under HIP
// graph capture, serving loops).  Every partial is written by the scan before
// the pick reads it, so the array needs no clearing.  One array per GPU,
// shared by every call on that GPU: calls that overlap on one GPU race.

namespace vt {

constexpr uint32_t NN_NOALLOC_MAX_QUERIES = 64;
static __device__ __align__(256) uint2 scratch[NN_NOALLOC_MAX_QUERIES * NN_SCAN_BLOCKS]; // 512 KiB

constexpr int NN_NOALLOC_MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static uint2 *g_scratch_ptr[NN_NOALLOC_MAX_DEVICES];

// Device address of the current device's copy of `scratch`, looked up once
// per device with that device current (host code never uses the symbol's
// host-side name as an address).
static int scratch_ptr_current_device(uint2 **out)
{
    int dev = -1;
    VT_HIP_CHECK(hipGetDevice(&dev));
    VT_REQUIRE(dev >= 0 && dev < NN_NOALLOC_MAX_DEVICES, "device ordinal %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        VT_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        VT_REQUIRE(p != nullptr, "scratch symbol has no device address");
        g_scratch_ptr[dev] = reinterpret_cast<uint2 *>(p);
    }
    *out = g_scratch_ptr[dev];
    return VT_OK;
}

} // namespace vt

extern "C" int vt_nearest_sites_noalloc(const float *points, uint32_t num_points, const float *queries,
                                        uint32_t num_queries, int32_t *out, vt_stream_t stream)
{
    clear_error();
    VT_REQUIRE(num_queries <= NN_NOALLOC_MAX_QUERIES,
               "vt_nearest_sites_noalloc: %u queries exceed its scratch capacity of %u queries", num_queries,
               NN_NOALLOC_MAX_QUERIES);
    if (num_queries) {
        VT_REQUIRE(num_points > 0, "no points to search");
        VT_REQUIRE(num_points < 0x7fffffffu, "too many points");
        VT_REQUIRE(points && queries && out, "null pointer argument");
    }
    // the address lookup comes before the zero-query return, so that a call
    // with no queries sets the device up (outside a graph capture) and
    // launches nothing
    uint2 *partial = nullptr;
    int rc = scratch_ptr_current_device(&partial);
    if (rc)
        return rc;
    if (num_queries == 0)
        return VT_OK;
    return launch_scan(points, num_points, queries, num_queries, partial, out, as_stream(stream));
}

extern "C" int vt_bvh_debug_stack_limit(void *handle, uint32_t limit, int force_tree)
{
    clear_error();
    BvhHandle *h = (BvhHandle *)handle;
    VT_REQUIRE(h, "null BVH handle");
    VT_REQUIRE(limit <= (uint32_t)BVH_STACK, "stack limit %u above the compiled %d", limit, BVH_STACK);
    h->stack_limit = limit ? limit : (uint32_t)BVH_STACK;
    h->force_tree = force_tree != 0;
    return VT_OK;
}

extern "C" int vt_bvh_num_nodes(void *handle)
{
    BvhHandle *h = (BvhHandle *)handle;
    return h ? (int)(h->n > 0 ? 2 * h->n - 1 : 0) : 0;
}
