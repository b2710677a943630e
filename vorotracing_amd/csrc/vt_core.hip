// vt_core.hip -- error state, the arithmetic self-test probe, and the
// per-face offset prefetch (tracing_octmap.cu:125-149, host :612-640).
#include "vt_internal.h"
#include "vt_device.h"
#include "vt_camera.h"
#include "vt_walk.h"

#include <cstring>

namespace vt {

static thread_local char g_err[1024];

void set_error(const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

void clear_error() { g_err[0] = 0; }

// op 6 rows: site p (3), origin o (3), unit direction d (3), face count nf
// (u32 bits; counts above 8 read as 8), then 8 face records (two u32 each)
// read as one chunk
constexpr int PROBE_FACE_ROW = 26;
constexpr int INFER_PROBE_CHUNK = 8;
// op 7 rows: an op 6 row whose records are in slot order (faces past nf are
// zero), then the slots' original indices as 8 u16 (4 words)
constexpr int PROBE_PACKED_ROW = 30;

__global__ void math_probe_kernel(int op, const float *__restrict__ in, uint32_t *__restrict__ out, uint32_t n)
{
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n)
        return;
    if (op == 5) { // in holds n records (num, dp, bnum, bdp)
        const float *r = in + 4 * (size_t)i;
        out[i] = exit_before(r[0], r[1], r[2], r[3]) ? 1u : 0u;
        return;
    }
    if (op == 6) { // in holds n rows of PROBE_FACE_ROW floats; out 2 words per row
        const float *r = in + PROBE_FACE_ROW * (size_t)i;
        const uint32_t nf = min(f_bits(r[9]), 8u); // the row holds 8 records
        float t1 = 0.0f;
        const uint32_t best = exit_face<INFER_PROBE_CHUNK>(reinterpret_cast<const uint2 *>(r + 10), nf,
                                                             mk(r[0], r[1], r[2]), mk(r[3], r[4], r[5]),
                                                             mk(r[6], r[7], r[8]), t1);
        out[2 * (size_t)i] = best;
        out[2 * (size_t)i + 1] = best == NONE ? 0u : f_bits(t1);
        return;
    }
    if (op == 7) { // the packed walk's search (walk_step_packed) over one reordered chunk; out (orig, t1 bits)
        const float *r = in + PROBE_PACKED_ROW * (size_t)i;
        const uint32_t *rec = reinterpret_cast<const uint32_t *>(r + 10);
        uint32_t h[24];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            h[3 * j] = rec[2 * j] & 0xffffu;
            h[3 * j + 1] = rec[2 * j] >> 16;
            h[3 * j + 2] = rec[2 * j + 1] & 0xffffu;
        }
        uint4 ch[3];
        uint32_t *cw = reinterpret_cast<uint32_t *>(ch);
#pragma unroll
        for (int k = 0; k < 12; ++k)
            cw[k] = h[2 * k] | h[2 * k + 1] << 16;
        uint16_t orig[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            orig[j] = (uint16_t)(f_bits(r[26 + j / 2]) >> (16 * (j & 1)));
        const f3 p = mk(r[0], r[1], r[2]), o = mk(r[3], r[4], r[5]), d = mk(r[6], r[7], r[8]);
        float bnum = FIRST_BNUM, bdp = FIRST_BDP;
        uint32_t best = NONE;
        search_chunk(ch[0], ch[1], ch[2], 0, p, o, d, bnum, bdp, best);
        float t1 = 0.0f;
        if (best != NONE) {
            t1 = bnum / bdp;
            if (!(t1 > -__builtin_huge_valf()))
                best = exit_face_packed_ieee(ch, 1, p, o, d, orig, t1);
        }
        out[2 * (size_t)i] = best == NONE ? NONE : orig[best];
        out[2 * (size_t)i + 1] = best == NONE ? 0u : f_bits(t1);
        return;
    }
    float x = in[i];
    if (op == 0)
        out[i] = f_bits(vt_expf(x));
    else if (op == 1)
        out[i] = f_bits(vt_logf(x));
    else if (op == 3)
        out[i] = f_bits(vt_sinf(x));
    else if (op == 4)
        out[i] = f_bits(vt_cosf(x));
    else
        out[i] = f2h(x);
}

// Prefetch: one block per 256 consecutive cells.  The block stages the
// cells' CSR offsets in LDS, then its lanes sweep the block's face entries
// with unit stride (coalesced adjacency reads and adj_diff writes).  The
// owning cell of an entry comes from a byte table in LDS that each lane
// fills for its cell's entries first (one LDS read per entry in the sweep);
// a block with more entries than the table holds (long hull-cell lists)
// finds it by binary search over the offsets.  Value per entry e of cell i:
// half(site[adj[e]] - site[i]) per axis (f32 subtract, RNE cast), w = 0.
constexpr int PF_CELLS = 256;
constexpr uint32_t PF_OWNER = 16384; // entries of a block whose owners fit the byte table

__global__ __launch_bounds__(PF_CELLS) void prefetch_kernel(const float *__restrict__ points, uint32_t num_points,
                                                             const uint32_t *__restrict__ adjacency,
                                                             const uint32_t *__restrict__ offsets,
                                                             uint2 *__restrict__ adj_diff)
{
    static_assert(PF_CELLS <= 256, "owners are stored as bytes");
    __shared__ uint32_t off[PF_CELLS + 1];
    __shared__ uint8_t owner[PF_OWNER];
    uint32_t c0 = blockIdx.x * PF_CELLS;
    uint32_t cnt = min((uint32_t)PF_CELLS, num_points - c0);
    for (uint32_t i = threadIdx.x; i <= cnt; i += blockDim.x)
        off[i] = offsets[c0 + i];
    __syncthreads();
    const uint32_t e0 = off[0], e1 = off[cnt];
    const bool table = e1 - e0 <= PF_OWNER; // block-uniform
    if (table) {
        for (uint32_t c = threadIdx.x; c < cnt; c += blockDim.x)
            for (uint32_t e = off[c]; e < off[c + 1]; ++e)
                owner[e - e0] = (uint8_t)c;
        __syncthreads();
    }
    for (uint32_t e = e0 + threadIdx.x; e < e1; e += blockDim.x) {
        uint32_t lo = 0;
        if (table) {
            lo = owner[e - e0];
        } else { // largest c with off[c] <= e (c < cnt)
            uint32_t hi = cnt;
            while (hi - lo > 1) {
                uint32_t mid = (lo + hi) >> 1;
                if (off[mid] <= e)
                    lo = mid;
                else
                    hi = mid;
            }
        }
        f3 p = load_site(points, c0 + lo);
        f3 q = load_site(points, adjacency[e]);
        f3 df = sub(q, p);
        uint2 w;
        w.x = (uint32_t)f2h(df.x) | ((uint32_t)f2h(df.y) << 16);
        w.y = (uint32_t)f2h(df.z);
        adj_diff[e] = w;
    }
}

// zero the rows past the last face list (the reference leaves them
// uninitialised; chunked face reads past a list end land here and are masked)
__global__ void zero_tail_kernel(const uint32_t *__restrict__ offsets, uint32_t num_points, uint32_t rows,
                                 uint2 *__restrict__ adj_diff)
{
    uint32_t start = offsets[num_points];
    for (uint32_t e = start + blockIdx.x * blockDim.x + threadIdx.x; e < rows; e += gridDim.x * blockDim.x)
        adj_diff[e] = make_uint2(0u, 0u);
}

int prefetch(const float *points, uint32_t num_points, const uint32_t *adjacency, uint32_t adjacency_size,
             const uint32_t *offsets, uint16_t *adj_diff, hipStream_t stream)
{
    VT_REQUIRE(points && adjacency && offsets && adj_diff, "null pointer argument");
    uint32_t rows = adjacency_size + 32;
    if (num_points > 0) {
        uint32_t blocks = (num_points + PF_CELLS - 1) / PF_CELLS;
        prefetch_kernel<<<blocks, PF_CELLS, 0, stream>>>(points, num_points, adjacency, offsets,
                                                         reinterpret_cast<uint2 *>(adj_diff));
        VT_LAUNCH_CHECK("prefetch_kernel");
    }
    zero_tail_kernel<<<4, 256, 0, stream>>>(offsets, num_points, rows, reinterpret_cast<uint2 *>(adj_diff));
    VT_LAUNCH_CHECK("zero_tail_kernel");
    return VT_OK;
}

} // namespace vt

using namespace vt;

extern "C" const char *vt_last_error(void) { return g_err; }

extern "C" int vt_abi_version(void) { return 12; }

extern "C" int vt_math_probe(int op, const float *in, uint32_t *out, uint32_t n, vt_stream_t stream)
{
    clear_error();
    VT_REQUIRE(op >= 0 && op <= 7,
               "op must be 0 (exp), 1 (log), 2 (f16), 3 (sin), 4 (cos), 5 (exit order), 6 (exit face) or 7 "
               "(packed exit face)");
    if (n == 0)
        return VT_OK;
    VT_REQUIRE(in && out, "null pointer argument");
    math_probe_kernel<<<(n + 255) / 256, 256, 0, as_stream(stream)>>>(op, in, out, n);
    VT_LAUNCH_CHECK("math_probe_kernel");
    return VT_OK;
}

extern "C" int vt_prefetch_adj(const float *points, uint32_t num_points, const uint32_t *adjacency,
                               uint32_t adjacency_size, const uint32_t *offsets, uint16_t *adj_diff,
                               vt_stream_t stream)
{
    clear_error();
    return prefetch(points, num_points, adjacency, adjacency_size, offsets, adj_diff, as_stream(stream));
}
