// vt_prep.hip -- preparation on the GPU: Morton reorder of cells with CSR
// rebuild (vorotracing.py:514-571), row permutation, screen-tile permutation
// (vorotracing.py:606-625), q8 quantisation and fp16 4-channel padding
// (vorotracing.py:495-512) for inference; the coherent lane order of flat
// training batches (vt_ray_order).
#include "vt_internal.h"
#include "vt_prims.h"
#include "vt_device.h"
#include "vt_walk.h"

namespace vt {

// 10-bit-per-axis Morton code with the reference's quantisation
// (vorotracing.py:519-530; same bit layout as geometry.h:271-283):
// q = trunc(clamp((p - lo) / max(hi - lo, 1e-6) * 1023, 0, 1023)).
__device__ __forceinline__ uint32_t morton10(f3 p, const float *bb)
{
    float v[3] = {p.x, p.y, p.z};
    uint32_t q[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        float size = __builtin_fmaxf(bb[3 + c] - bb[c], 1e-6f);
        float x = ((v[c] - bb[c]) / size) * 1023.0f;
        x = __builtin_fminf(__builtin_fmaxf(x, 0.0f), 1023.0f);
        q[c] = (uint32_t)x;
    }
    uint32_t code = 0;
#pragma unroll
    for (int i = 0; i < 10; ++i) {
        code |= ((q[0] >> i) & 1u) << (3 * i);
        code |= ((q[1] >> i) & 1u) << (3 * i + 1);
        code |= ((q[2] >> i) & 1u) << (3 * i + 2);
    }
    return code;
}

__global__ void morton_keys_kernel(const float *__restrict__ points, uint32_t n, const float *__restrict__ bb,
                                   uint32_t *__restrict__ keys, uint32_t *__restrict__ vals)
{
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n)
        return;
    keys[i] = morton10(load_site(points, i), bb);
    vals[i] = i;
}

// new cell i = old cell perm[i]
__global__ void morton_gather_kernel(const uint32_t *__restrict__ perm, uint32_t n, const float *__restrict__ points,
                                     const uint32_t *__restrict__ offsets, float *__restrict__ points_out,
                                     uint32_t *__restrict__ inv_perm, uint32_t *__restrict__ counts)
{
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i > n)
        return;
    if (i == n) {
        counts[n] = 0;
        return;
    }
    uint32_t o = perm[i];
    inv_perm[o] = i;
    f3 p = load_site(points, o);
    points_out[3 * (size_t)i + 0] = p.x;
    points_out[3 * (size_t)i + 1] = p.y;
    points_out[3 * (size_t)i + 2] = p.z;
    counts[i] = offsets[o + 1] - offsets[o];
}

// Copy each face list to its new place, preserving intra-list order and
// remapping neighbour ids through inv_perm.  One block per 256 new cells;
// entries swept with unit stride, owner found by binary search in LDS.
constexpr int CP_CELLS = 256;

__global__ __launch_bounds__(CP_CELLS) void morton_copy_lists_kernel(
    const uint32_t *__restrict__ perm, const uint32_t *__restrict__ inv_perm, uint32_t n,
    const uint32_t *__restrict__ offsets, const uint32_t *__restrict__ adjacency,
    const uint32_t *__restrict__ new_offsets, uint32_t *__restrict__ adjacency_out)
{
    __shared__ uint32_t off[CP_CELLS + 1];
    __shared__ uint32_t src[CP_CELLS];
    uint32_t c0 = blockIdx.x * CP_CELLS;
    uint32_t cnt = min((uint32_t)CP_CELLS, n - c0);
    for (uint32_t i = threadIdx.x; i <= cnt; i += blockDim.x)
        off[i] = new_offsets[c0 + i];
    for (uint32_t i = threadIdx.x; i < cnt; i += blockDim.x)
        src[i] = offsets[perm[c0 + i]];
    __syncthreads();
    uint32_t e0 = off[0], e1 = off[cnt];
    for (uint32_t e = e0 + threadIdx.x; e < e1; e += blockDim.x) {
        uint32_t lo = 0, hi = cnt;
        while (hi - lo > 1) {
            uint32_t mid = (lo + hi) >> 1;
            if (off[mid] <= e)
                lo = mid;
            else
                hi = mid;
        }
        adjacency_out[e] = inv_perm[adjacency[src[lo] + (e - off[lo])]];
    }
}

__global__ void zero_u32_from_kernel(const uint32_t *__restrict__ start_at, uint32_t end, uint32_t *__restrict__ a)
{
    uint32_t s = *start_at;
    for (uint32_t e = s + blockIdx.x * blockDim.x + threadIdx.x; e < end; e += gridDim.x * blockDim.x)
        a[e] = 0;
}

// dst row i = src row perm[i]; rows of `row_bytes` bytes
__global__ void permute_rows_kernel(const uint8_t *__restrict__ src, uint32_t rows, uint32_t row_bytes,
                                    const uint32_t *__restrict__ perm, uint8_t *__restrict__ dst, int vec)
{
    size_t total_units = (size_t)rows * (row_bytes / vec);
    size_t units_per_row = row_bytes / vec;
    for (size_t u = (size_t)blockIdx.x * blockDim.x + threadIdx.x; u < total_units;
         u += (size_t)gridDim.x * blockDim.x) {
        size_t r = u / units_per_row, k = u % units_per_row;
        size_t so = (size_t)perm[r] * row_bytes + k * vec, dofs = r * row_bytes + k * vec;
        if (vec == 16)
            *reinterpret_cast<uint4 *>(dst + dofs) = *reinterpret_cast<const uint4 *>(src + so);
        else if (vec == 4)
            *reinterpret_cast<uint32_t *>(dst + dofs) = *reinterpret_cast<const uint32_t *>(src + so);
        else
            dst[dofs] = src[so];
    }
}

// perm[rank] = pixel, rank = position of the pixel's key
// ((y/TH)*ceil(W/TW) + x/TW)*TH*TW + (y%TH)*TW + x%TW among all keys
// (vorotracing.py:618-623); partial edge tiles are compacted as argsort does.
__global__ void tile_perm_kernel(uint32_t H, uint32_t W, uint32_t TH, uint32_t TW, int32_t *__restrict__ perm)
{
    uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= H * W)
        return;
    uint32_t y = p / W, x = p % W;
    uint32_t ty = y / TH, tx = x / TW;
    uint32_t h = min(TH, H - ty * TH), w = min(TW, W - tx * TW);
    uint32_t rank = ty * TH * W + h * tx * TW + (y % TH) * w + (x % TW);
    perm[rank] = (int32_t)p;
}

// --- coherent lane order for flat ray batches --------------------------------

// Direction bits per octahedral axis of the order key: a 128 x 128 grid over
// the sphere, cells of about 1.4 degrees.  With the start cell's bits the key
// then fits one word up to 2^18 sites (one sort instead of two).  Random
// pixels of 32 cameras over C2's scene: forward + backward 3.34-3.39 ms
// against 3.44-3.56 with 8 bits and 3.57-3.60 with 10.
#ifndef VT_ORDER_DIR_BITS
#define VT_ORDER_DIR_BITS 7
#endif
constexpr int ORDER_DIR_BITS = VT_ORDER_DIR_BITS;

__device__ __forceinline__ uint32_t spread_bits(uint32_t x) // bit i -> bit 2i (x < 2^16)
{
    x &= 0xffffu;
    x = (x | (x << 8)) & 0x00ff00ffu;
    x = (x | (x << 4)) & 0x0f0f0f0fu;
    x = (x | (x << 2)) & 0x33333333u;
    x = (x | (x << 1)) & 0x55555555u;
    return x;
}

// 2-D Morton code of the ray direction's octahedral coordinates: nearby
// directions get nearby keys.  A NaN coordinate clamps to cell 0.
__device__ __forceinline__ uint32_t direction_key(const float *__restrict__ rays, uint32_t i)
{
    const float dx = rays[6 * (size_t)i + 3], dy = rays[6 * (size_t)i + 4], dz = rays[6 * (size_t)i + 5];
    const float l1 = __builtin_fmaxf(__builtin_fabsf(dx) + __builtin_fabsf(dy) + __builtin_fabsf(dz), 1e-30f);
    float u = dx / l1, v = dy / l1;
    if (dz < 0.0f) {
        const float ou = (1.0f - __builtin_fabsf(v)) * __builtin_copysignf(1.0f, u);
        const float ov = (1.0f - __builtin_fabsf(u)) * __builtin_copysignf(1.0f, v);
        u = ou;
        v = ov;
    }
    constexpr float cells = (float)(1u << ORDER_DIR_BITS);
    const float top = cells - 1.0f;
    const uint32_t qu = (uint32_t)__builtin_fminf(__builtin_fmaxf((u * 0.5f + 0.5f) * cells, 0.0f), top);
    const uint32_t qv = (uint32_t)__builtin_fminf(__builtin_fmaxf((v * 0.5f + 0.5f) * cells, 0.0f), top);
    return spread_bits(qu) | (spread_bits(qv) << 1);
}

// keys[i] = (start cell << 2*ORDER_DIR_BITS) | direction key when both fit
// one word (cell_shift > 0), else the direction key alone; vals[i] = i.
__global__ void ray_order_keys_kernel(const float *__restrict__ rays, const uint32_t *__restrict__ start_point,
                                      uint32_t n, int cell_shift, uint32_t *__restrict__ keys,
                                      uint32_t *__restrict__ vals)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n)
        return;
    uint32_t k = direction_key(rays, i);
    if (cell_shift)
        k |= start_point[i] << cell_shift;
    keys[i] = k;
    vals[i] = i;
}

// keys[j] = start cell of ray vals[j] (the second, stable pass of a two-pass order)
__global__ void ray_order_cells_kernel(const uint32_t *__restrict__ start_point, const uint32_t *__restrict__ vals,
                                       uint32_t n, uint32_t *__restrict__ keys)
{
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j < n)
        keys[j] = start_point[vals[j]];
}

// --- q8 quantisation ---------------------------------------------------------

// ws[0..2] min, ws[3..5] max (ordered ints), per channel or all in channel 0
__global__ __launch_bounds__(256) void minmax_kernel(const float *__restrict__ x, size_t n, int per_channel,
                                                     int32_t *ws)
{
    int32_t lo[3] = {0x7fffffff, 0x7fffffff, 0x7fffffff};
    int32_t hi[3] = {(int32_t)0x80000000, (int32_t)0x80000000, (int32_t)0x80000000};
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        int c = per_channel ? (int)(i % 3) : 0;
        int32_t o = f2ord(x[i]);
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            if (k == c) {
                lo[k] = min(lo[k], o);
                hi[k] = max(hi[k], o);
            }
        }
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) {
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            lo[k] = min(lo[k], __shfl_xor(lo[k], o, 64));
            hi[k] = max(hi[k], __shfl_xor(hi[k], o, 64));
        }
    }
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            atomicMin(ws + k, lo[k]);
            atomicMax(ws + 3 + k, hi[k]);
        }
    }
}

__global__ void minmax_init_kernel(int32_t *ws)
{
    if (threadIdx.x < 3)
        ws[threadIdx.x] = 0x7fffffff;
    else if (threadIdx.x < 6)
        ws[threadIdx.x] = (int32_t)0x80000000;
}

// scale = fp32((double(vmax) - double(vmin)) / 255), offset = vmin
// (vorotracing.py:498-501); params = {scale[3], offset[3], inv_scale[3]}
__global__ void q8_params_kernel(const int32_t *ws, int per_channel, float *params)
{
    int c = threadIdx.x;
    if (c >= 3)
        return;
    int k = per_channel ? c : 0;
    float vmin = ord2f(ws[k]), vmax = ord2f(ws[3 + k]);
    float scale = (float)(((double)vmax - (double)vmin) / 255.0);
    params[c] = scale;
    params[3 + c] = vmin;
    params[6 + c] = 1.0f / scale;
}

// q = clamp(rint((x - offset) * fp32(1/scale)), 0, 255): torch's CUDA
// true-division by a CPU scalar multiplies by the fp32 reciprocal
__global__ void q8_apply_kernel(const float *__restrict__ x, size_t n, int per_channel,
                                const float *__restrict__ params, uint8_t *__restrict__ q)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        int c = per_channel ? (int)(i % 3) : 0;
        float scale = params[c];
        float v = 0.0f;
        if (scale != 0.0f) {
            v = __builtin_rintf((x[i] - params[3 + c]) * params[6 + c]);
            v = __builtin_fminf(__builtin_fmaxf(v, 0.0f), 255.0f);
        }
        q[i] = (uint8_t)v;
    }
}

// (rows, 3*RR) f32 -> (rows, 4*RR) f16 with zero 4th channel (RNE cast)
__global__ void pad34_kernel(const float *__restrict__ x, size_t texels, uint2 *__restrict__ out)
{
    for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < texels; t += (size_t)gridDim.x * blockDim.x) {
        const float *s = x + 3 * t;
        uint2 w;
        w.x = (uint32_t)f2h(s[0]) | ((uint32_t)f2h(s[1]) << 16);
        w.y = (uint32_t)f2h(s[2]);
        out[t] = w;
    }
}

static uint32_t grid_for(size_t n, uint32_t block = 256, uint32_t cap = 8192)
{
    size_t g = (n + block - 1) / block;
    return (uint32_t)(g < 1 ? 1 : (g > cap ? cap : g));
}

} // namespace vt

using namespace vt;

// words: keys n, vals n, inv n, counts n+1, sort ws, scan ws (n+1), bbox 6+6
static size_t morton_ws_words(uint32_t n)
{
    return 4 * (size_t)n + 1 + radix_sort_workspace_words(n) + scan_workspace_words(n + 1) + 16;
}

extern "C" size_t vt_morton_workspace_size(uint32_t num_points, uint32_t adjacency_size)
{
    (void)adjacency_size;
    return morton_ws_words(num_points) * 4;
}

extern "C" int vt_morton_reorder(const float *points, uint32_t num_points, const uint32_t *adjacency,
                                 uint32_t adjacency_size, const uint32_t *offsets, uint32_t *perm,
                                 float *points_out, uint32_t *adjacency_out, uint32_t *offsets_out,
                                 void *workspace, vt_stream_t stream)
{
    clear_error();
    VT_REQUIRE(points && adjacency && offsets && perm && points_out && adjacency_out && offsets_out && workspace,
               "null pointer argument");
    const uint32_t adj_out_size = adjacency_size;
    hipStream_t s = as_stream(stream);
    uint32_t n = num_points;
    if (n == 0) {
        zero_u32_from_kernel<<<1, 64, 0, s>>>(offsets, adj_out_size, adjacency_out);
        VT_LAUNCH_CHECK("zero_u32_from_kernel");
        VT_HIP_CHECK(hipMemcpyAsync(offsets_out, offsets, 4, hipMemcpyDeviceToDevice, s));
        return VT_OK;
    }
    uint32_t *w = (uint32_t *)workspace;
    uint32_t *keys = w;
    uint32_t *vals = keys + n;
    uint32_t *inv = vals + n;
    uint32_t *counts = inv + n;
    uint32_t *sws = counts + n + 1;
    uint32_t *scan_ws = sws + radix_sort_workspace_words(n);
    uint32_t *bbw = scan_ws + scan_workspace_words(n + 1);
    float *bb = (float *)(bbw + 8);
    int rc = bbox3(points, n, bb, bbw, s);
    if (rc)
        return rc;
    morton_keys_kernel<<<(n + 255) / 256, 256, 0, s>>>(points, n, bb, keys, vals);
    VT_LAUNCH_CHECK("morton_keys_kernel");
    rc = radix_sort_pairs(keys, vals, n, 30, sws, s);
    if (rc)
        return rc;
    VT_HIP_CHECK(hipMemcpyAsync(perm, vals, (size_t)n * 4, hipMemcpyDeviceToDevice, s));
    morton_gather_kernel<<<(n + 1 + 255) / 256, 256, 0, s>>>(perm, n, points, offsets, points_out, inv, counts);
    VT_LAUNCH_CHECK("morton_gather_kernel");
    rc = exclusive_scan_u32(counts, offsets_out, n + 1, scan_ws, s);
    if (rc)
        return rc;
    morton_copy_lists_kernel<<<(n + CP_CELLS - 1) / CP_CELLS, CP_CELLS, 0, s>>>(perm, inv, n, offsets, adjacency,
                                                                               offsets_out, adjacency_out);
    VT_LAUNCH_CHECK("morton_copy_lists_kernel");
    zero_u32_from_kernel<<<4, 256, 0, s>>>(offsets_out + n, adj_out_size, adjacency_out);
    VT_LAUNCH_CHECK("zero_u32_from_kernel");
    return VT_OK;
}

extern "C" int vt_permute_rows(const void *src, uint32_t rows, uint32_t row_bytes, const uint32_t *perm, void *dst,
                               vt_stream_t stream)
{
    clear_error();
    if (rows == 0 || row_bytes == 0)
        return VT_OK;
    VT_REQUIRE(src && perm && dst && src != dst, "null or aliased pointer argument");
    int vec = (row_bytes % 16 == 0 && ((uintptr_t)src % 16 == 0) && ((uintptr_t)dst % 16 == 0)) ? 16
              : (row_bytes % 4 == 0 && ((uintptr_t)src % 4 == 0) && ((uintptr_t)dst % 4 == 0)) ? 4
                                                                                                 : 1;
    size_t units = (size_t)rows * (row_bytes / vec);
    permute_rows_kernel<<<grid_for(units), 256, 0, as_stream(stream)>>>((const uint8_t *)src, rows, row_bytes, perm,
                                                                        (uint8_t *)dst, vec);
    VT_LAUNCH_CHECK("permute_rows_kernel");
    return VT_OK;
}

extern "C" int vt_tile_perm(uint32_t height, uint32_t width, uint32_t tile_h, uint32_t tile_w, int32_t *perm,
                            vt_stream_t stream)
{
    clear_error();
    VT_REQUIRE(tile_h > 0 && tile_w > 0, "tile sizes must be positive");
    VT_REQUIRE((uint64_t)height * width < (1ull << 31), "image too large");
    if (height == 0 || width == 0)
        return VT_OK;
    VT_REQUIRE(perm, "null pointer argument");
    uint32_t n = height * width;
    tile_perm_kernel<<<(n + 255) / 256, 256, 0, as_stream(stream)>>>(height, width, tile_h, tile_w, perm);
    VT_LAUNCH_CHECK("tile_perm_kernel");
    return VT_OK;
}

// ---- launch order of screen tiles ------------------------------------------

namespace vt {

// Key of the stable ascending sort that lists tiles by decreasing cost: the
// cost's octave and its next three bits, 8 buckets per doubling over costs
// 16 to 2^20 (costs below share the last bucket, costs above the first; 7
// bits), inverted.  Within a bucket tiles keep screen order, so the blocks an
// XCD takes in one turn still cover neighbouring tiles and share their cells
// in that XCD's L2.  4 buckets per octave left the frame's last tiles in a
// worse order (C3 same view 1.723 against 1.703 ms); 16 gained no more.
constexpr uint32_t TILE_ORDER_FRAC = 3;
constexpr uint32_t TILE_ORDER_LB0 = 4;
constexpr uint32_t TILE_ORDER_OCTAVES = 16;
constexpr uint32_t TILE_ORDER_TOP = (TILE_ORDER_OCTAVES << TILE_ORDER_FRAC) - 1u;

__host__ __device__ constexpr uint32_t tile_order_key(uint32_t cost)
{
    const uint32_t c = cost > 1u ? cost : 1u;
    const uint32_t lb = 31u - (uint32_t)__builtin_clz(c);
    if (lb < TILE_ORDER_LB0)
        return TILE_ORDER_TOP;
    if (lb >= TILE_ORDER_LB0 + TILE_ORDER_OCTAVES)
        return 0u;
    const uint32_t frac = (c >> (lb - TILE_ORDER_FRAC)) & ((1u << TILE_ORDER_FRAC) - 1u);
    return TILE_ORDER_TOP - (((lb - TILE_ORDER_LB0) << TILE_ORDER_FRAC) | frac);
}
static_assert(TILE_ORDER_LB0 >= TILE_ORDER_FRAC, "the fraction bits lie below the octave bit");
static_assert(TILE_ORDER_TOP < 128, "keys fit 7 bits: the scatter ranks them by 7 ballots");
static_assert(tile_order_key(1) == TILE_ORDER_TOP && tile_order_key(0) == TILE_ORDER_TOP &&
                  tile_order_key(15) == TILE_ORDER_TOP && tile_order_key(16) == TILE_ORDER_TOP,
              "");
static_assert(tile_order_key(0xffffffffu) == 0 && tile_order_key(1u << 20) == 0, "");
static_assert(tile_order_key(24) < tile_order_key(20) && tile_order_key(20) < tile_order_key(18), "");
static_assert(tile_order_key(1000) == tile_order_key(1023) && tile_order_key(1023) > tile_order_key(1024), "");

// The order is a stable counting sort of the keys (TILE_ORDER_TOP + 1 bins)
// in three launches: per-block key histograms and cost sums; one block that
// scans the histograms bin-major (each block's first position per key) and
// totals the costs; and a stable scatter, in which each block also counts
// its tiles above the split share into tile_order[tiles].
constexpr uint32_t TO_BLOCK = 256; // tiles per block
constexpr uint32_t TO_BINS = TILE_ORDER_TOP + 1;
constexpr uint32_t TO_SCAN_THREADS = 1024;
static_assert(TO_BINS <= TO_BLOCK, "one thread per bin");

__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, uint64_t *red)
{
    red[threadIdx.x] = v;
    __syncthreads();
    for (uint32_t h = blockDim.x / 2; h > 0; h >>= 1) {
        if (threadIdx.x < h)
            red[threadIdx.x] += red[threadIdx.x + h];
        __syncthreads();
    }
    const uint64_t total = red[0];
    __syncthreads();
    return total;
}

// hist[bin * blocks + block] = tiles of the block with that key; psum[block]
// = the block's cost sum
__global__ __launch_bounds__(TO_BLOCK) void tile_hist_kernel(const uint32_t *__restrict__ cost, uint32_t tiles,
                                                             uint32_t *__restrict__ hist, uint64_t *__restrict__ psum)
{
    __shared__ uint32_t h[TO_BINS];
    __shared__ uint64_t red[TO_BLOCK];
    if (threadIdx.x < TO_BINS)
        h[threadIdx.x] = 0;
    __syncthreads();
    const uint32_t t = blockIdx.x * TO_BLOCK + threadIdx.x;
    const uint32_t c = t < tiles ? cost[t] : 0u;
    if (t < tiles)
        atomicAdd(&h[tile_order_key(c)], 1u);
    const uint64_t sum = block_sum_u64(c, red);
    if (threadIdx.x < TO_BINS)
        hist[threadIdx.x * gridDim.x + blockIdx.x] = h[threadIdx.x];
    if (threadIdx.x == 0)
        psum[blockIdx.x] = sum;
}

// One block: hist scanned in place (exclusive, bin-major), *total = the sum
// of psum, *split = 0
__global__ __launch_bounds__(TO_SCAN_THREADS) void tile_scan_kernel(uint32_t *__restrict__ hist, uint32_t n,
                                                                    const uint64_t *__restrict__ psum, uint32_t blocks,
                                                                    uint64_t *__restrict__ total,
                                                                    uint32_t *__restrict__ split)
{
    __shared__ uint32_t wsum[TO_SCAN_THREADS / 64];
    __shared__ uint64_t red[TO_SCAN_THREADS];
    const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
    uint32_t carry = 0;
    for (uint32_t base = 0; base < n; base += TO_SCAN_THREADS) {
        const uint32_t i = base + threadIdx.x;
        const uint32_t v = i < n ? hist[i] : 0u;
        uint32_t x = v; // inclusive scan within the wave
#pragma unroll
        for (uint32_t o = 1; o < 64; o <<= 1) {
            const uint32_t y = __shfl_up(x, o, 64);
            if (lane >= o)
                x += y;
        }
        if (lane == 63)
            wsum[w] = x;
        __syncthreads();
        uint32_t before = carry;
        for (uint32_t j = 0; j < w; ++j)
            before += wsum[j];
        uint32_t chunk = 0;
        for (uint32_t j = 0; j < TO_SCAN_THREADS / 64; ++j)
            chunk += wsum[j];
        if (i < n)
            hist[i] = before + x - v;
        carry += chunk;
        __syncthreads();
    }
    uint64_t sum = 0;
    for (uint32_t b = threadIdx.x; b < blocks; b += TO_SCAN_THREADS)
        sum += psum[b];
    sum = block_sum_u64(sum, red);
    if (threadIdx.x == 0) {
        *total = sum;
        *split = 0u;
    }
}

// Stable scatter: tile t to its key's next position, tiles of a block in
// order (lanes, then waves, through 7 key-bit ballots and per-wave counts).
// A tile is split when its cost exceeds SPLIT_NUM / SPLIT_DEN of the mean
// load of one resident wave (total cost / split_waves): such a tile, started
// first, still runs when the launch's other work has drained, and the
// launch ends with it.  Tiles below that are covered by the other waves.
constexpr uint64_t SPLIT_NUM = 4, SPLIT_DEN = 5;

__global__ __launch_bounds__(TO_BLOCK) void tile_scatter_kernel(const uint32_t *__restrict__ cost, uint32_t tiles,
                                                                const uint32_t *__restrict__ hist,
                                                                const uint64_t *__restrict__ total,
                                                                uint32_t split_waves, uint32_t *__restrict__ order)
{
    __shared__ uint32_t base[TO_BINS];
    __shared__ uint32_t wcnt[TO_BLOCK / 64][TO_BINS];
    __shared__ uint32_t nsplit;
    if (threadIdx.x < TO_BINS) {
        base[threadIdx.x] = hist[threadIdx.x * gridDim.x + blockIdx.x];
#pragma unroll
        for (uint32_t j = 0; j < TO_BLOCK / 64; ++j)
            wcnt[j][threadIdx.x] = 0;
    }
    if (threadIdx.x == 0)
        nsplit = 0;
    __syncthreads();
    const uint32_t t = blockIdx.x * TO_BLOCK + threadIdx.x;
    const bool valid = t < tiles;
    const uint32_t c = valid ? cost[t] : 0u;
    const uint32_t key = tile_order_key(c);
    const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
    uint64_t m = __ballot(valid);
#pragma unroll
    for (uint32_t b = 0; b < 7; ++b) {
        const bool bit = (key >> b) & 1u;
        const uint64_t bb = __ballot(bit);
        m &= bit ? bb : ~bb;
    }
    const uint64_t lt = lane ? (~0ull >> (64 - lane)) : 0ull;
    const uint32_t rank = (uint32_t)__popcll(m & lt);
    if (valid && rank == 0)
        wcnt[w][key] = (uint32_t)__popcll(m);
    // (the left side stays below 2^59: cost < 2^32, split_waves < 2^24; a
    // total of 2^57 or more splits nothing and would overflow on the right)
    const uint64_t tot = *total;
    if (valid && split_waves && tot < (1ull << 57) && SPLIT_DEN * (uint64_t)c * split_waves > SPLIT_NUM * tot)
        atomicAdd(&nsplit, 1u);
    __syncthreads();
    if (valid) {
        uint32_t pos = base[key] + rank;
        for (uint32_t j = 0; j < w; ++j)
            pos += wcnt[j][key];
        order[pos] = t;
    }
    if (threadIdx.x == 0 && nsplit)
        atomicAdd(order + tiles, nsplit);
}

} // namespace vt

static uint32_t tile_order_blocks(uint32_t tiles) { return (tiles + TO_BLOCK - 1) / TO_BLOCK; }

// workspace: hist (TO_BINS words per block), psum (one u64 per block), total (u64)
extern "C" size_t vt_tile_order_workspace_size(uint32_t tiles)
{
    const size_t blocks = tile_order_blocks(tiles);
    return (blocks * TO_BINS * 4 + 7) / 8 * 8 + (blocks + 1) * 8;
}

extern "C" int vt_tile_order(const uint32_t *tile_cost, uint32_t tiles, uint32_t split_waves, uint32_t *tile_order,
                             void *workspace, vt_stream_t stream)
{
    clear_error();
    if (tiles == 0)
        return VT_OK;
    VT_REQUIRE(tile_cost && tile_order && workspace, "null pointer argument");
    VT_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 8 == 0, "workspace must be 8-byte aligned");
    VT_REQUIRE(split_waves < (1u << 24), "split_waves (%u) must be below 2^24", split_waves);
    hipStream_t s = as_stream(stream);
    const uint32_t blocks = tile_order_blocks(tiles);
    uint32_t *hist = static_cast<uint32_t *>(workspace);
    uint64_t *psum = reinterpret_cast<uint64_t *>(static_cast<char *>(workspace) +
                                                  ((size_t)blocks * TO_BINS * 4 + 7) / 8 * 8);
    uint64_t *total = psum + blocks;
    tile_hist_kernel<<<blocks, TO_BLOCK, 0, s>>>(tile_cost, tiles, hist, psum);
    VT_LAUNCH_CHECK("tile_hist_kernel");
    tile_scan_kernel<<<1, TO_SCAN_THREADS, 0, s>>>(hist, blocks * TO_BINS, psum, blocks, total, tile_order + tiles);
    VT_LAUNCH_CHECK("tile_scan_kernel");
    tile_scatter_kernel<<<blocks, TO_BLOCK, 0, s>>>(tile_cost, tiles, hist, total, split_waves, tile_order);
    VT_LAUNCH_CHECK("tile_scatter_kernel");
    return VT_OK;
}

extern "C" size_t vt_ray_order_workspace_size(uint32_t num_rays)
{
    return ((size_t)num_rays + radix_sort_workspace_words(num_rays)) * 4;
}

extern "C" int vt_ray_order(const float *rays, const uint32_t *start_point, uint32_t num_rays, uint32_t num_points,
                            uint32_t *ray_perm, void *workspace, vt_stream_t stream)
{
    clear_error();
    if (num_rays == 0)
        return VT_OK;
    VT_REQUIRE(rays && start_point && ray_perm && workspace, "null pointer argument");
    VT_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 4 == 0, "workspace must be 4-byte aligned");
    hipStream_t s = as_stream(stream);
    uint32_t *keys = static_cast<uint32_t *>(workspace);
    uint32_t *sws = keys + num_rays;
    const int dir_bits = 2 * ORDER_DIR_BITS;
    const int cell_bits = num_points > 1 ? 32 - __builtin_clz(num_points - 1) : 0;
    const uint32_t blocks = (num_rays + 255) / 256;
    if (cell_bits + dir_bits <= 32) {
        ray_order_keys_kernel<<<blocks, 256, 0, s>>>(rays, start_point, num_rays, cell_bits ? dir_bits : 0, keys,
                                                     ray_perm);
        VT_LAUNCH_CHECK("ray_order_keys_kernel");
        return radix_sort_pairs(keys, ray_perm, num_rays, cell_bits + dir_bits, sws, s);
    }
    // Direction first, then a stable sort by start cell: cell-major order.
    ray_order_keys_kernel<<<blocks, 256, 0, s>>>(rays, start_point, num_rays, 0, keys, ray_perm);
    VT_LAUNCH_CHECK("ray_order_keys_kernel");
    int rc = radix_sort_pairs(keys, ray_perm, num_rays, dir_bits, sws, s);
    if (rc)
        return rc;
    ray_order_cells_kernel<<<blocks, 256, 0, s>>>(start_point, ray_perm, num_rays, keys);
    VT_LAUNCH_CHECK("ray_order_cells_kernel");
    return radix_sort_pairs(keys, ray_perm, num_rays, cell_bits, sws, s);
}

extern "C" size_t vt_quantize_workspace_size(void) { return 64; }

// x f32 (rows, cols) with cols % 3 == 0 when per_channel; params out (device,
// 9 floats: scale[3], offset[3], 1/scale[3]); ws: vt_quantize_workspace_size bytes
extern "C" int vt_quantize_u8(const float *x, uint32_t rows, uint32_t cols, int per_channel, uint8_t *q,
                              float *params, void *workspace, vt_stream_t stream)
{
    clear_error();
    VT_REQUIRE(x && q && params && workspace, "null pointer argument");
    VT_REQUIRE(!per_channel || cols % 3 == 0, "per-channel quantisation needs RGB-interleaved columns");
    hipStream_t s = as_stream(stream);
    size_t n = (size_t)rows * cols;
    int32_t *ws = (int32_t *)workspace;
    minmax_init_kernel<<<1, 64, 0, s>>>(ws);
    VT_LAUNCH_CHECK("minmax_init_kernel");
    if (n > 0) {
        minmax_kernel<<<grid_for(n, 256, 2048), 256, 0, s>>>(x, n, per_channel, ws);
        VT_LAUNCH_CHECK("minmax_kernel");
    }
    q8_params_kernel<<<1, 64, 0, s>>>(ws, per_channel, params);
    VT_LAUNCH_CHECK("q8_params_kernel");
    if (n > 0) {
        q8_apply_kernel<<<grid_for(n), 256, 0, s>>>(x, n, per_channel, params, q);
        VT_LAUNCH_CHECK("q8_apply_kernel");
    }
    return VT_OK;
}

extern "C" int vt_pad_3to4_f16(const float *x, uint32_t rows, uint32_t texels_per_row, uint16_t *out,
                               vt_stream_t stream)
{
    clear_error();
    VT_REQUIRE(x && out, "null pointer argument");
    size_t t = (size_t)rows * texels_per_row;
    if (t == 0)
        return VT_OK;
    pad34_kernel<<<grid_for(t), 256, 0, as_stream(stream)>>>(x, t, reinterpret_cast<uint2 *>(out));
    VT_LAUNCH_CHECK("pad34_kernel");
    return VT_OK;
}

// ---------------------------------------------------------------------------
// Packed walk layout (vt_walk_layout): the inference walk's arrays regrouped
// so that a step issues fewer vector loads (the walk side is in vt_walk.h).

namespace vt {

__global__ void wl_init_kernel(uint32_t *first_chunk, uint32_t n)
{
    if (blockIdx.x == 0 && threadIdx.x == 0)
        first_chunk[n + 1] = 0;
}

// chunk count of each cell (8 faces per chunk); [n] = 0 so that the scan
// leaves the total there; [n + 1] = the largest count
// One lane per cell: its chunk count, and whether its list holds a
// neighbour id at or past n (bit 31 of first_chunk[n + 1], which no count
// reaches).
__global__ void wl_count_kernel(const uint32_t *offsets, const uint32_t *adjacency, uint32_t n,
                                uint32_t *first_chunk)
{
    const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t k = 0, bad = 0;
    if (c < n) {
        const uint32_t b = offsets[c], e = offsets[c + 1];
        k = (uint32_t)(((uint64_t)e - b + 7u) >> 3);
        first_chunk[c] = k;
        for (uint32_t f = b; f < e; ++f)
            bad |= adjacency[f] >= n ? 1u : 0u;
    } else if (c == n) {
        first_chunk[n] = 0;
    }
    // one atomic per wave for the largest count (and the flag)
    k = wave_max_u32(k | bad << 31);
    if ((threadIdx.x & 63u) == 0 && k)
        atomicMax(first_chunk + n + 1, k);
}

// Lists of up to WL_SORT_MAX faces are laid out in the face order; longer
// ones (hull cells) keep theirs.
constexpr uint32_t WL_SORT_MAX = 64;

// The face order's key of f16 bits h: a total order that is the numeric one
// on non-NaN values, with -0 taken as +0 and NaNs past the infinities of
// their sign.
__device__ __forceinline__ uint32_t face_order_key(uint32_t h)
{
    h = h == 0x8000u ? 0u : h;
    return (h & 0x8000u) ? 0x7fffu - (h & 0x7fffu) : (h | 0x8000u);
}

// One lane per cell: its cell record, its head, and its chunks, links and
// original indices.  face_order 1..3 sorts the cell's faces by the
// face_order_key of the x, y or z half of their offsets (equal keys keep list
// order), 0 keeps the list order.  The sort ranks (key, index) pairs, which
// are distinct, so the ranks are a permutation of the list.
__global__ void wl_fill_kernel(const float *__restrict__ points, const float *__restrict__ density,
                               const uint32_t *__restrict__ adjacency, const uint32_t *__restrict__ offsets,
                               uint32_t n, const uint2 *__restrict__ adj_diff, const uint32_t *__restrict__ fc,
                               int face_order, uint4 *__restrict__ chunks, uint2 *__restrict__ links,
                               uint2 *__restrict__ heads, float4 *__restrict__ cells, uint16_t *__restrict__ origs)
{
    const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= n)
        return;
    const uint32_t b = offsets[c], nf = offsets[c + 1] - b;
    const uint32_t cb = fc[c], nch = fc[c + 1] - cb;
    const f3 p = load_site(points, c);
    cells[c] = make_float4(p.x, p.y, p.z, density[c]);
    heads[c] = make_uint2(c | nch << WL_ID_BITS, cb);
    uint16_t ord[WL_SORT_MAX];
    const bool sorted = face_order >= 1 && face_order <= 3 && nf <= WL_SORT_MAX;
    if (sorted) {
        // (key << 8 | index) per face, loaded once; a face's slot is the
        // number of smaller pairs
        uint32_t kv[WL_SORT_MAX];
        for (uint32_t f = 0; f < nf; ++f) {
            const uint2 r = adj_diff[b + f];
            const uint32_t h = face_order == 1 ? (r.x & 0xffffu) : face_order == 2 ? (r.x >> 16) : (r.y & 0xffffu);
            kv[f] = face_order_key(h) << 8 | f;
        }
        for (uint32_t f = 0; f < nf; ++f) {
            uint32_t rank = 0;
            for (uint32_t g = 0; g < nf; ++g)
                rank += kv[g] < kv[f] ? 1u : 0u;
            ord[rank] = (uint16_t)f;
        }
    }
    for (uint32_t q = 0; q < nch; ++q) {
        // the chunk's 24 halves: x, y, z of face 0, then of face 1, ...
        uint32_t w[12] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t slot = 8 * q + j;
            uint2 lk = make_uint2(0u, 0u);
            uint16_t og = 0xffffu;
            if (slot < nf) {
                const uint32_t f = sorted ? ord[slot] : slot;
                const uint2 r = adj_diff[b + f];
                const uint32_t h[3] = {r.x & 0xffffu, r.x >> 16, r.y & 0xffffu};
#pragma unroll
                for (int a = 0; a < 3; ++a) {
                    const int k = 3 * j + a;
                    w[k >> 1] |= h[a] << (16 * (k & 1));
                }
                // an id out of range (flagged by vt_walk_layout_count) links the cell to itself
                const uint32_t nb = adjacency[b + f] < n ? adjacency[b + f] : c;
                const uint32_t ncb = fc[nb];
                lk = make_uint2(nb | (fc[nb + 1] - ncb) << WL_ID_BITS, ncb);
                og = (uint16_t)f;
            }
            links[8 * (size_t)(cb + q) + j] = lk;
            origs[8 * (size_t)(cb + q) + j] = og;
        }
        uint4 *row = chunks + 3 * (size_t)(cb + q);
        row[0] = make_uint4(w[0], w[1], w[2], w[3]);
        row[1] = make_uint4(w[4], w[5], w[6], w[7]);
        row[2] = make_uint4(w[8], w[9], w[10], w[11]);
    }
}

// Footprint tables of fp16 octahedral maps (vt_quad_maps): one lane per
// (cell, entry); entry (ex, ey) holds the wrapped texels of the taps
// (ex - 1, ey - 1), (ex, ey - 1), (ex - 1, ey), (ex, ey), the ones
// bilinear_setup reads for floor coordinates (ex - 1, ey - 1).  Coordinates
// stay in [-1, R], the range oct_wrap_edge reduces.
// The q8 footprint tables: as quad_maps_kernel below, each texel's three bytes
// widened to one (r, g, b, 0) word, an entry one 16-byte word.
template <int R>
__global__ void quad_maps_q8_kernel(const uint8_t *__restrict__ maps, uint32_t n, uint4 *__restrict__ quads)
{
    constexpr uint32_t E = (R + 1) * (R + 1);
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)n * E)
        return;
    const uint64_t c = i / E;
    const int e = (int)(i - c * E);
    const int ex = e % (R + 1), ey = e / (R + 1);
    const uint8_t *m = maps + c * (3 * R * R);
    auto texel = [&](int t) {
        return (uint32_t)m[3 * t] | (uint32_t)m[3 * t + 1] << 8 | (uint32_t)m[3 * t + 2] << 16;
    };
    quads[i] = make_uint4(texel(oct_wrap_edge<R>(ex - 1, ey - 1)), texel(oct_wrap_edge<R>(ex, ey - 1)),
                          texel(oct_wrap_edge<R>(ex - 1, ey)), texel(oct_wrap_edge<R>(ex, ey)));
}

template <int R>
__global__ void quad_maps_kernel(const uint2 *__restrict__ maps, uint32_t n, uint4 *__restrict__ quads)
{
    constexpr uint32_t E = (R + 1) * (R + 1);
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)n * E)
        return;
    const uint64_t c = i / E;
    const int e = (int)(i - c * E);
    const int ex = e % (R + 1), ey = e / (R + 1);
    const uint2 *m = maps + c * (R * R);
    const uint2 t00 = m[oct_wrap_edge<R>(ex - 1, ey - 1)], t10 = m[oct_wrap_edge<R>(ex, ey - 1)];
    const uint2 t01 = m[oct_wrap_edge<R>(ex - 1, ey)], t11 = m[oct_wrap_edge<R>(ex, ey)];
    quads[2 * i] = make_uint4(t00.x, t00.y, t10.x, t10.y);
    quads[2 * i + 1] = make_uint4(t01.x, t01.y, t11.x, t11.y);
}

} // namespace vt

extern "C" size_t vt_walk_layout_count_workspace_size(uint32_t num_points)
{
    return 4 * scan_workspace_words(num_points + 1);
}

extern "C" int vt_walk_layout_count(const uint32_t *offsets, const uint32_t *adjacency, uint32_t num_points,
                                    uint32_t *first_chunk, void *ws, vt_stream_t stream)
{
    clear_error();
    VT_REQUIRE(offsets && adjacency && first_chunk && ws, "null pointer argument");
    VT_REQUIRE(num_points < 0xffffffffu, "too many points");
    hipStream_t s = as_stream(stream);
    wl_init_kernel<<<1, 64, 0, s>>>(first_chunk, num_points);
    VT_LAUNCH_CHECK("wl_init_kernel");
    wl_count_kernel<<<(uint32_t)(((size_t)num_points + 256) / 256), 256, 0, s>>>(offsets, adjacency, num_points,
                                                                              first_chunk);
    VT_LAUNCH_CHECK("wl_count_kernel");
    return exclusive_scan_u32(first_chunk, first_chunk, num_points + 1, (uint32_t *)ws, s);
}

extern "C" int vt_walk_layout_fill(const float *points, const float *density, const uint32_t *adjacency,
                                   const uint32_t *offsets, uint32_t num_points, const uint16_t *adj_diff,
                                   const uint32_t *first_chunk, uint32_t num_chunks, int face_order,
                                   uint32_t *chunks, uint32_t *links, uint32_t *heads, float *cells, uint16_t *orig,
                                   vt_stream_t stream)
{
    clear_error();
    VT_REQUIRE(points && density && adjacency && offsets && adj_diff && first_chunk && chunks && links && heads &&
                   cells && orig,
               "null pointer argument");
    VT_REQUIRE(face_order >= 0 && face_order <= 3, "face_order must be 0 (list order), 1, 2 or 3 (x, y, z), got %d",
               face_order);
    VT_REQUIRE(num_points < (1u << WL_ID_BITS), "the walk layout holds cell ids below 2^24, got %u points",
               num_points);
    VT_REQUIRE(num_chunks < (1u << 29), "the walk layout holds fewer than 2^29 chunks, got %u", num_chunks);
    if (num_points == 0)
        return VT_OK;
    wl_fill_kernel<<<(num_points + 255) / 256, 256, 0, as_stream(stream)>>>(
        points, density, adjacency, offsets, num_points, reinterpret_cast<const uint2 *>(adj_diff), first_chunk,
        face_order, reinterpret_cast<uint4 *>(chunks), reinterpret_cast<uint2 *>(links),
        reinterpret_cast<uint2 *>(heads), reinterpret_cast<float4 *>(cells), orig);
    VT_LAUNCH_CHECK("wl_fill_kernel");
    return VT_OK;
}

extern "C" int vt_quad_maps_f16(const uint16_t *maps, uint32_t num_points, uint32_t res, uint16_t *quads,
                                vt_stream_t stream)
{
    clear_error();
    VT_REQUIRE(res == 4 || res == 8, "res must be 4 or 8, got %u", res);
    if (num_points == 0)
        return VT_OK;
    VT_REQUIRE(maps && quads, "null pointer argument");
    VT_REQUIRE((reinterpret_cast<uintptr_t>(maps) & 7u) == 0 && (reinterpret_cast<uintptr_t>(quads) & 15u) == 0,
               "maps must be 8-byte and quads 16-byte aligned");
    const uint64_t lanes = (uint64_t)num_points * (res + 1) * (res + 1);
    const uint64_t blocks = (lanes + 255) / 256;
    VT_REQUIRE(blocks < (1ull << 31), "too many cells for one launch: %u", num_points);
    if (res == 4)
        quad_maps_kernel<4><<<(uint32_t)blocks, 256, 0, as_stream(stream)>>>(
            reinterpret_cast<const uint2 *>(maps), num_points, reinterpret_cast<uint4 *>(quads));
    else
        quad_maps_kernel<8><<<(uint32_t)blocks, 256, 0, as_stream(stream)>>>(
            reinterpret_cast<const uint2 *>(maps), num_points, reinterpret_cast<uint4 *>(quads));
    VT_LAUNCH_CHECK("quad_maps_kernel");
    return VT_OK;
}

extern "C" int vt_quad_maps_q8(const uint8_t *maps, uint32_t num_points, uint32_t res, uint8_t *quads,
                               vt_stream_t stream)
{
    clear_error();
    VT_REQUIRE(res == 4 || res == 8, "res must be 4 or 8, got %u", res);
    if (num_points == 0)
        return VT_OK;
    VT_REQUIRE(maps && quads, "null pointer argument");
    VT_REQUIRE((reinterpret_cast<uintptr_t>(quads) & 15u) == 0, "quads must be 16-byte aligned");
    const uint64_t lanes = (uint64_t)num_points * (res + 1) * (res + 1);
    const uint64_t blocks = (lanes + 255) / 256;
    VT_REQUIRE(blocks < (1ull << 31), "too many cells for one launch: %u", num_points);
    if (res == 4)
        quad_maps_q8_kernel<4><<<(uint32_t)blocks, 256, 0, as_stream(stream)>>>(maps, num_points,
                                                                               reinterpret_cast<uint4 *>(quads));
    else
        quad_maps_q8_kernel<8><<<(uint32_t)blocks, 256, 0, as_stream(stream)>>>(maps, num_points,
                                                                               reinterpret_cast<uint4 *>(quads));
    VT_LAUNCH_CHECK("quad_maps_q8_kernel");
    return VT_OK;
}
