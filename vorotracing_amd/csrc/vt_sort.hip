// vt_sort.hip -- exclusive scan, stable LSD radix sort (8-bit digits) and
// point bounding box.  Tiles are 256 lanes x 16 items; wave-level ranking uses
// 64-lane ballots.
#include "vt_internal.h"
#include "vt_prims.h"

namespace vt {

constexpr int P_THREADS = 256;
constexpr int P_ITEMS = 16;
constexpr uint32_t P_TILE = P_THREADS * P_ITEMS;
constexpr int P_WAVES = P_THREADS / 64;

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v)
{
    int lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        uint32_t t = __shfl_up(v, o, 64);
        if (lane >= o)
            v += t;
    }
    return v;
}

// exclusive scan of one value per lane over the block; total of the block out
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t *lds, uint32_t &total)
{
    uint32_t incl = wave_incl_scan(v);
    int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 63)
        lds[w] = incl;
    __syncthreads();
    uint32_t pre = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < P_WAVES; ++i) {
        uint32_t x = lds[i];
        pre += (i < w) ? x : 0u;
        tot += x;
    }
    __syncthreads();
    total = tot;
    return pre + incl - v;
}

__global__ __launch_bounds__(P_THREADS) void scan_reduce_kernel(const uint32_t *__restrict__ in, uint32_t n,
                                                                 uint32_t *__restrict__ partials)
{
    __shared__ uint32_t lds[P_WAVES];
    uint32_t base = blockIdx.x * P_TILE;
    uint32_t s = 0;
    for (int k = 0; k < P_ITEMS; ++k) {
        uint32_t i = base + k * P_THREADS + threadIdx.x;
        if (i < n)
            s += in[i];
    }
    uint32_t total;
    block_excl_scan(s, lds, total);
    if (threadIdx.x == 0)
        partials[blockIdx.x] = total;
}

// thread t owns items [base + 16 t, base + 16 t + 16)
__global__ __launch_bounds__(P_THREADS) void scan_apply_kernel(const uint32_t *in, uint32_t *out, uint32_t n,
                                                                const uint32_t *__restrict__ partials)
{
    __shared__ uint32_t lds[P_WAVES];
    uint32_t base = blockIdx.x * P_TILE + threadIdx.x * P_ITEMS;
    uint32_t v[P_ITEMS];
    uint32_t s = 0;
#pragma unroll
    for (int k = 0; k < P_ITEMS; ++k) {
        uint32_t i = base + k;
        v[k] = (i < n) ? in[i] : 0u;
        s += v[k];
    }
    uint32_t total;
    uint32_t run = block_excl_scan(s, lds, total) + (partials ? partials[blockIdx.x] : 0u);
#pragma unroll
    for (int k = 0; k < P_ITEMS; ++k) {
        uint32_t i = base + k;
        if (i < n)
            out[i] = run;
        run += v[k];
    }
}

size_t scan_workspace_words(uint32_t n)
{
    if (n <= P_TILE)
        return 0;
    uint32_t t = (n + P_TILE - 1) / P_TILE;
    return t + scan_workspace_words(t);
}

int exclusive_scan_u32(const uint32_t *in, uint32_t *out, uint32_t n, uint32_t *ws, hipStream_t s)
{
    if (n == 0)
        return VT_OK;
    if (n <= P_TILE) {
        scan_apply_kernel<<<1, P_THREADS, 0, s>>>(in, out, n, nullptr);
        VT_LAUNCH_CHECK("scan_apply_kernel");
        return VT_OK;
    }
    uint32_t t = (n + P_TILE - 1) / P_TILE;
    scan_reduce_kernel<<<t, P_THREADS, 0, s>>>(in, n, ws);
    VT_LAUNCH_CHECK("scan_reduce_kernel");
    int rc = exclusive_scan_u32(ws, ws, t, ws + t, s);
    if (rc)
        return rc;
    scan_apply_kernel<<<t, P_THREADS, 0, s>>>(in, out, n, ws);
    VT_LAUNCH_CHECK("scan_apply_kernel");
    return VT_OK;
}

// ---------------------------------------------------------------------------
// radix sort

// hist[d * tiles + tile] = count of digit d in the tile
__global__ __launch_bounds__(P_THREADS) void radix_hist_kernel(const uint32_t *__restrict__ keys, uint32_t n,
                                                                int shift, uint32_t *__restrict__ hist,
                                                                uint32_t tiles)
{
    __shared__ uint32_t cnt[256];
    cnt[threadIdx.x] = 0;
    __syncthreads();
    uint32_t base = blockIdx.x * P_TILE;
    for (int k = 0; k < P_ITEMS; ++k) {
        uint32_t i = base + k * P_THREADS + threadIdx.x;
        if (i < n)
            atomicAdd(&cnt[(keys[i] >> shift) & 255u], 1u);
    }
    __syncthreads();
    hist[threadIdx.x * tiles + blockIdx.x] = cnt[threadIdx.x];
}

// Stable scatter: items are taken in 16 rounds of 256 consecutive keys; in a
// round, the rank of a key among equal digits is (keys of that digit in
// earlier waves) + (in earlier lanes of its wave, from 8 digit-bit ballots).
__global__ __launch_bounds__(P_THREADS) void radix_scatter_kernel(const uint32_t *__restrict__ kin,
                                                                   const uint32_t *__restrict__ vin,
                                                                   uint32_t *__restrict__ kout,
                                                                   uint32_t *__restrict__ vout, uint32_t n,
                                                                   int shift, const uint32_t *__restrict__ hist,
                                                                   uint32_t tiles)
{
    __shared__ uint32_t base_d[256];
    __shared__ uint32_t wcnt[P_WAVES][256];
    base_d[threadIdx.x] = hist[threadIdx.x * tiles + blockIdx.x];
    const int w = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    uint32_t tile_base = blockIdx.x * P_TILE;
    for (int k = 0; k < P_ITEMS; ++k) {
#pragma unroll
        for (int j = 0; j < P_WAVES; ++j)
            wcnt[j][threadIdx.x] = 0;
        __syncthreads();
        uint32_t i = tile_base + k * P_THREADS + threadIdx.x;
        bool valid = i < n;
        uint32_t key = valid ? kin[i] : 0u;
        uint32_t val = valid ? vin[i] : 0u;
        uint32_t d = (key >> shift) & 255u;
        uint64_t m = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            bool bit = (d >> b) & 1u;
            uint64_t bb = __ballot(bit);
            m &= bit ? bb : ~bb;
        }
        uint32_t rank = (uint32_t)__popcll(m & lt);
        if (valid && rank == 0)
            wcnt[w][d] = (uint32_t)__popcll(m);
        __syncthreads();
        if (valid) {
            uint32_t off = base_d[d] + rank;
            for (int j = 0; j < w; ++j)
                off += wcnt[j][d];
            kout[off] = key;
            vout[off] = val;
        }
        __syncthreads();
        uint32_t add = 0;
#pragma unroll
        for (int j = 0; j < P_WAVES; ++j)
            add += wcnt[j][threadIdx.x];
        base_d[threadIdx.x] += add;
        __syncthreads();
    }
}

size_t radix_pass_workspace_words(uint32_t n)
{
    uint32_t tiles = (n + P_TILE - 1) / P_TILE;
    return 256 * (size_t)tiles + scan_workspace_words(256 * tiles);
}

int radix_sort_pass(const uint32_t *kin, const uint32_t *vin, uint32_t *kout, uint32_t *vout, uint32_t n, int shift,
                    uint32_t *ws, hipStream_t s)
{
    if (n == 0)
        return VT_OK;
    uint32_t tiles = (n + P_TILE - 1) / P_TILE;
    uint32_t *hist = ws;
    uint32_t *sws = hist + 256 * (size_t)tiles;
    radix_hist_kernel<<<tiles, P_THREADS, 0, s>>>(kin, n, shift, hist, tiles);
    VT_LAUNCH_CHECK("radix_hist_kernel");
    int rc = exclusive_scan_u32(hist, hist, 256 * tiles, sws, s);
    if (rc)
        return rc;
    radix_scatter_kernel<<<tiles, P_THREADS, 0, s>>>(kin, vin, kout, vout, n, shift, hist, tiles);
    VT_LAUNCH_CHECK("radix_scatter_kernel");
    return VT_OK;
}

size_t radix_sort_workspace_words(uint32_t n)
{
    return 2 * (size_t)n + radix_pass_workspace_words(n);
}

int radix_sort_pairs(uint32_t *keys, uint32_t *vals, uint32_t n, int bits, uint32_t *ws, hipStream_t s)
{
    if (n <= 1)
        return VT_OK;
    uint32_t *k2 = ws;
    uint32_t *v2 = ws + n;
    uint32_t *pws = ws + 2 * (size_t)n;
    int passes = (bits + 7) / 8;
    uint32_t *ka = keys, *va = vals, *kb = k2, *vb = v2;
    for (int p = 0; p < passes; ++p) {
        int rc = radix_sort_pass(ka, va, kb, vb, n, 8 * p, pws, s);
        if (rc)
            return rc;
        uint32_t *t = ka;
        ka = kb;
        kb = t;
        t = va;
        va = vb;
        vb = t;
    }
    if (ka != keys) {
        VT_HIP_CHECK(hipMemcpyAsync(keys, ka, (size_t)n * 4, hipMemcpyDeviceToDevice, s));
        VT_HIP_CHECK(hipMemcpyAsync(vals, va, (size_t)n * 4, hipMemcpyDeviceToDevice, s));
    }
    return VT_OK;
}

// ---------------------------------------------------------------------------
// bounding box

__global__ void bbox_init_kernel(int32_t *ws)
{
    if (threadIdx.x < 3)
        ws[threadIdx.x] = 0x7fffffff;
    else if (threadIdx.x < 6)
        ws[threadIdx.x] = (int32_t)0x80000000;
}

__global__ __launch_bounds__(256) void bbox_reduce_kernel(const float *__restrict__ p, uint32_t n, int32_t *ws)
{
    int32_t lo[3] = {0x7fffffff, 0x7fffffff, 0x7fffffff};
    int32_t hi[3] = {(int32_t)0x80000000, (int32_t)0x80000000, (int32_t)0x80000000};
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            int32_t o = f2ord(p[3 * (size_t)i + c]);
            lo[c] = min(lo[c], o);
            hi[c] = max(hi[c], o);
        }
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) {
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            lo[c] = min(lo[c], __shfl_xor(lo[c], o, 64));
            hi[c] = max(hi[c], __shfl_xor(hi[c], o, 64));
        }
    }
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            atomicMin(ws + c, lo[c]);
            atomicMax(ws + 3 + c, hi[c]);
        }
    }
}

__global__ void bbox_final_kernel(const int32_t *ws, float *bbox6)
{
    if (threadIdx.x < 6)
        bbox6[threadIdx.x] = ord2f(ws[threadIdx.x]);
}

int bbox3(const float *points, uint32_t n, float *bbox6, uint32_t *ws, hipStream_t s)
{
    bbox_init_kernel<<<1, 64, 0, s>>>((int32_t *)ws);
    VT_LAUNCH_CHECK("bbox_init_kernel");
    if (n > 0) {
        uint32_t blocks = min((n + 255u) / 256u, 1024u);
        bbox_reduce_kernel<<<blocks, 256, 0, s>>>(points, n, (int32_t *)ws);
        VT_LAUNCH_CHECK("bbox_reduce_kernel");
    }
    bbox_final_kernel<<<1, 64, 0, s>>>((const int32_t *)ws, bbox6);
    VT_LAUNCH_CHECK("bbox_final_kernel");
    return VT_OK;
}

} // namespace vt
