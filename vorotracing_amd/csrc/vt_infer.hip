// vt_infer.hip -- inference traversal: fp16 Half4Texel and q8 attribute
// integrators (ray_integrator_octmap.cuh:295-633), their kernels
// (tracing_octmap.cu:552-610, :723-779) and C entry points.
//
// One lane per ray.  The integrators advance transmittance only for cells
// with density > 1e-6, shade a cell only when its weight reaches the skip
// threshold, and stop once T <= weight_threshold.
//
// Shading is deferred: about half the lanes of a wave shade in a given step,
// so shading in place would run its ~250 instructions at half the lanes.
// The integrator queues (cell, weight, offset to the probe point) in the
// wave's LDS ring instead; when 64 entries wait, every lane shades one, and
// each ray then adds its results in queue order, i.e. in its own step order,
// so the colour sums are the same operations in the same order as in place.
// The colour of a cell uses approximate arithmetic (shade_sigmoid below).
#include "vt_internal.h"
#include "vt_walk.h"
#include "vt_camera.h"

#include <algorithm>

namespace vt {

// fp16 Half4Texel maps: texel = 8 bytes (r, g, b, pad) halves.  QUADS: the
// maps' footprint tables (vt_quad_maps) are read instead, a tap's four texels
// as one 32-byte entry (two 16-byte loads in one cache line) instead of four
// 8-byte texels; the texels and weights are the same, so is the colour.
template <int RD, int RS, bool QUADS> struct TexF16 {
    const uint2 *diffuse;  // maps, or footprint tables (QUADS)
    const uint2 *specular;

    __device__ __forceinline__ static constexpr bool quads() { return QUADS; }
    __device__ __forceinline__ f3 sample_diffuse(uint32_t cell, const Bilinear &b) const
    {
        if constexpr (QUADS)
            return sample_quad(reinterpret_cast<const uint4 *>(diffuse) +
                                   2 * ((size_t)cell * ((RD + 1) * (RD + 1)) + (uint32_t)b.i00),
                               b);
        else
            return sample(diffuse + (size_t)cell * (RD * RD), b);
    }
    __device__ __forceinline__ f3 sample_specular(uint32_t cell, const Bilinear &b) const
    {
        if constexpr (QUADS)
            return sample_quad(reinterpret_cast<const uint4 *>(specular) +
                                   2 * ((size_t)cell * ((RS + 1) * (RS + 1)) + (uint32_t)b.i00),
                               b);
        else
            return sample(specular + (size_t)cell * (RS * RS), b);
    }
    __device__ __forceinline__ static f3 mix(const Bilinear &b, uint2 a, uint2 c, uint2 e, uint2 g)
    {
        float r = bil_mix(b, h2f(a.x & 0xffffu), h2f(c.x & 0xffffu), h2f(e.x & 0xffffu), h2f(g.x & 0xffffu));
        float gg = bil_mix(b, h2f(a.x >> 16), h2f(c.x >> 16), h2f(e.x >> 16), h2f(g.x >> 16));
        float bl = bil_mix(b, h2f(a.y & 0xffffu), h2f(c.y & 0xffffu), h2f(e.y & 0xffffu), h2f(g.y & 0xffffu));
        return mk(r, gg, bl);
    }
    __device__ __forceinline__ static f3 sample(const uint2 *m, const Bilinear &b)
    {
        return mix(b, m[b.i00], m[b.i10], m[b.i01], m[b.i11]);
    }
    // entry: texels (u0, v0), (u0 + 1, v0) | (u0, v0 + 1), (u0 + 1, v0 + 1)
    __device__ __forceinline__ static f3 sample_quad(const uint4 *m, const Bilinear &b)
    {
        const uint4 p0 = m[0], p1 = m[1];
        return mix(b, make_uint2(p0.x, p0.y), make_uint2(p0.z, p0.w), make_uint2(p1.x, p1.y),
                   make_uint2(p1.z, p1.w));
    }
};

// q8 maps: texel = 3 bytes, dequant = scale[c] * q + offset[c].  QUADS: the
// maps' q8 footprint tables (vt_quad_maps) are read instead, a tap's four
// texels (r, g, b, 0 bytes each) as one 16-byte entry instead of twelve single
// bytes; the bytes and weights are the same, so is the colour.
template <int RD, int RS, bool QUADS> struct TexQ8 {
    const uint8_t *diffuse; // maps, or footprint tables (QUADS)
    const uint8_t *specular;
    float ds[3], dof[3], ss[3], sof[3];

    __device__ __forceinline__ static constexpr bool quads() { return QUADS; }
    __device__ __forceinline__ f3 sample_diffuse(uint32_t cell, const Bilinear &b) const
    {
        if constexpr (QUADS)
            return sample_quad(reinterpret_cast<const uint4 *>(diffuse)[(size_t)cell * ((RD + 1) * (RD + 1)) +
                                                                         (uint32_t)b.i00],
                               b, ds, dof);
        else
            return sample(diffuse + (size_t)cell * (3 * RD * RD), b, ds, dof);
    }
    __device__ __forceinline__ f3 sample_specular(uint32_t cell, const Bilinear &b) const
    {
        if constexpr (QUADS)
            return sample_quad(reinterpret_cast<const uint4 *>(specular)[(size_t)cell * ((RS + 1) * (RS + 1)) +
                                                                          (uint32_t)b.i00],
                               b, ss, sof);
        else
            return sample(specular + (size_t)cell * (3 * RS * RS), b, ss, sof);
    }
    // entry words: texels (u0, v0), (u0 + 1, v0), (u0, v0 + 1), (u0 + 1, v0 + 1)
    __device__ __forceinline__ static f3 sample_quad(uint4 e, const Bilinear &b, const float *sc, const float *of)
    {
        float v[3];
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            float a = fma_(sc[c], (float)((e.x >> (8 * c)) & 0xffu), of[c]);
            float bb = fma_(sc[c], (float)((e.y >> (8 * c)) & 0xffu), of[c]);
            float cc = fma_(sc[c], (float)((e.z >> (8 * c)) & 0xffu), of[c]);
            float d = fma_(sc[c], (float)((e.w >> (8 * c)) & 0xffu), of[c]);
            v[c] = bil_mix(b, a, bb, cc, d);
        }
        return mk(v[0], v[1], v[2]);
    }
    __device__ __forceinline__ static f3 sample(const uint8_t *m, const Bilinear &b, const float *sc,
                                                const float *of)
    {
        float v[3];
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            float a = fma_(sc[c], (float)m[b.i00 * 3 + c], of[c]);
            float bb = fma_(sc[c], (float)m[b.i10 * 3 + c], of[c]);
            float cc = fma_(sc[c], (float)m[b.i01 * 3 + c], of[c]);
            float d = fma_(sc[c], (float)m[b.i11 * 3 + c], of[c]);
            v[c] = bil_mix(b, a, bb, cc, d);
        }
        return mk(v[0], v[1], v[2]);
    }
};

// One wave per block: a block's LDS queue is freed as soon as its wave ends.
// With 4-wave blocks the LDS of 8 blocks filled a CU, so a block whose other
// waves had ended kept a new one from starting until its last wave ended.
constexpr int INFER_BLOCK = 64;
constexpr int INFER_CHUNK = 8;
// Blocks per XCD turn (xcd_interleaved_block): with contiguous ranges per XCD
// (xcd_block) one XCD got the costliest screen region and finished last.
constexpr uint32_t INFER_XCD_CHUNK = 32;



// The pending shades of one wave: a ring of SQ_RING entries.  Lanes append
// from inside the integrator (at most 64 per walk step); the wave shades
// 64 at a time at the uniform point after a step (an entry's colour then
// replaces its dv).  Plus each lane's specular taps, fixed per ray.
constexpr uint32_t SQ_RING = 128;
struct ShadeQueue {
    uint32_t cell[SQ_RING];
    float w[SQ_RING], dvx[SQ_RING], dvy[SQ_RING], dvz[SQ_RING];
    uint8_t owner[SQ_RING];          // owner lane | 0x80 when dv is already the direction
    unsigned long long mask[64];     // per owner lane: its entries in the batch
    uint32_t si[64];                 // specular taps, 8 bits each
    float sw[4][64];                 // specular weights (tap-major: lanes of different owners on different banks)
    uint32_t tail;                   // entries appended so far (mod 2^32)
};
__shared__ ShadeQueue infer_queues[INFER_BLOCK / 64];

__device__ __forceinline__ ShadeQueue &wave_queue() { return infer_queues[threadIdx.x >> 6]; }

// RayIntegratorOctMapInfer / ...InferQ8 (ray_integrator_octmap.cuh:315-344,
// :487-515, colour :437-460).  A cell to shade goes to the wave's queue as
// (cell, weight, probe offset); shade_batch computes its colour.
template <int RD, int RS, class Tex> struct InferIntegrator {
    using TexType = Tex;
    f3 o, d;
    const float *density;
    Tex tex;
    float thr, skip;
    f3 acc;
    float T;
    float pdens; // density of the current cell, loaded by begin_cell

    __device__ __forceinline__ void begin_cell(uint32_t cell) { pdens = density[cell]; }
    // the density when the walk state carries it (packed walk layout)
    __device__ __forceinline__ void begin_cell_value(float dens) { pdens = dens; }

    template <class S>
    __device__ __forceinline__ bool integrate(uint32_t cell, float t0, float t1, f3 p, f3, S &st)
    {
        float s = pdens;
        if (s <= 1e-6f)
            return T > thr;
        float dt = __builtin_fmaxf(t1 - t0, 0.0f);
        float alpha = 1.0f - vt_expf(-s * dt);
        float w = T * alpha;
        if (w >= skip) {
            st.shade();
            // probe_dir's test len > 1e-8 on the squared length (exact, see PROBE_LEN2_MIN)
            const f3 dv = sub(mk(fma_(t0, d.x, o.x), fma_(t0, d.y, o.y), fma_(t0, d.z, o.z)), p);
            const bool tiny = !(dot(dv, dv) > PROBE_LEN2_MIN);
            // the lanes appending now are exactly the active ones
            ShadeQueue &q = wave_queue();
            const uint64_t m = __ballot(1);
            const uint32_t rank = lane_rank(m), tail = q.tail;
            const uint32_t k = (tail + rank) & (SQ_RING - 1);
            q.cell[k] = cell;
            q.w[k] = w;
            // component selects: a select of the two structs would take their
            // addresses and push the integrator into scratch memory
            q.dvx[k] = tiny ? d.x : dv.x;
            q.dvy[k] = tiny ? d.y : dv.y;
            q.dvz[k] = tiny ? d.z : dv.z;
            q.owner[k] = (uint8_t)((threadIdx.x & 63u) | (tiny ? 0x80u : 0u));
            if (rank == 0)
                q.tail = tail + (uint32_t)__popcll(m);
        }
        T = T * (1.0f - alpha);
        return T > thr;
    }
};

// Colour arithmetic of the inference kernels.  It feeds only the RGB sums,
// so it uses the hardware approximations v_rsq_f32, v_rcp_f32 and v_exp_f32
// (each within about 1 ulp) in place of the correctly rounded sqrt, divisions
// and vt_expf.  The colours of a shaded cell then move by about 1e-6 of their
// range, and the fp16 RGB output by at most one fp16 ulp (4.9e-4 near 1): the
// required bound is 2e-3.  Everything that decides the walk (exit faces,
// t1, alpha, transmittance, the skip gate) stays exact, so visit sequences and
// the alpha channel remain bit-identical to the CPU checker.  The training
// kernels keep exact colours: their gradients are checked to 1e-3.
__device__ __forceinline__ float shade_sigmoid(float x)
{
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504f));
}

// oct_encode with 1/l1 by v_rcp_f32.  |x| <= l1, so |u|, |v| <= 1 + 2^-21 and
// the bilinear taps stay in the [-1, R] range oct_wrap_edge reduces.
template <int R> __device__ __forceinline__ void shade_oct_encode(f3 d, float &tu, float &tv)
{
    const float l1 = (__builtin_fabsf(d.x) + __builtin_fabsf(d.y)) + __builtin_fabsf(d.z);
    const float inv = __builtin_amdgcn_rcpf(l1);
    float u = d.x * inv;
    float v = d.y * inv;
    if (d.z < 0.0f) {
        const float ou = (1.0f - __builtin_fabsf(v)) * __builtin_copysignf(1.0f, u);
        const float ov = (1.0f - __builtin_fabsf(u)) * __builtin_copysignf(1.0f, v);
        u = ou;
        v = ov;
    }
    tu = fma_(fma_(u, 0.5f, 0.5f), (float)R, -0.5f);
    tv = fma_(fma_(v, 0.5f, 0.5f), (float)R, -0.5f);
}

// Shade entries [head, head + nb) of the ring, one per lane (probe_dir,
// octahedral lookup of the diffuse map, the ray's specular taps, sigmoid),
// then each owner adds its entries' colours in ring order.
template <int RD, int RS, class Integ>
__device__ __forceinline__ void shade_batch(ShadeQueue &q, uint32_t head, uint32_t nb, Integ &integ, int lane)
{
    static_assert(RS * RS <= 256, "specular tap indices are stored as bytes");
    if ((uint32_t)lane < nb) {
        const uint32_t k = (head + (uint32_t)lane) & (SQ_RING - 1);
        const uint32_t ob = q.owner[k], own = ob & 63u;
        const f3 dv = mk(q.dvx[k], q.dvy[k], q.dvz[k]);
        // |dv|^2 > PROBE_LEN2_MIN (about 1e-16) here, or dv is the unit direction
        const float il = (ob & 0x80u) ? 1.0f : __builtin_amdgcn_rsqf(dot(dv, dv));
        const f3 pd = mk(dv.x * il, dv.y * il, dv.z * il);
        float u, v;
        shade_oct_encode<RD>(pd, u, v);
        Bilinear db;
        if constexpr (Integ::TexType::quads())
            db = bilinear_quad<RD>(u, v);
        else
            db = bilinear_setup<RD>(u, v);
        Bilinear sb;
        const uint32_t si = q.si[own];
        if constexpr (Integ::TexType::quads()) { // the footprint entry
            sb.i00 = (int)si;
            sb.i10 = sb.i01 = sb.i11 = 0;
        } else {
            sb.i00 = (int)(si & 0xffu);
            sb.i10 = (int)((si >> 8) & 0xffu);
            sb.i01 = (int)((si >> 16) & 0xffu);
            sb.i11 = (int)(si >> 24);
        }
        sb.w00 = q.sw[0][own];
        sb.w10 = q.sw[1][own];
        sb.w01 = q.sw[2][own];
        sb.w11 = q.sw[3][own];
        const uint32_t cell = q.cell[k];
        const f3 a = integ.tex.sample_diffuse(cell, db);
        const f3 b = integ.tex.sample_specular(cell, sb);
        const f3 lg = add(a, b);
        q.dvx[k] = shade_sigmoid(lg.x);
        q.dvy[k] = shade_sigmoid(lg.y);
        q.dvz[k] = shade_sigmoid(lg.z);
        atomicOr(&q.mask[own], 1ull << lane);
    }
    wave_lds_sync();
    unsigned long long m = q.mask[lane];
    if (m) {
        q.mask[lane] = 0ull;
        do {
            const int i = __ffsll(m) - 1;
            m &= m - 1;
            const uint32_t k = (head + (uint32_t)i) & (SQ_RING - 1);
            integ.acc = vfma(q.w[k], mk(q.dvx[k], q.dvy[k], q.dvz[k]), integ.acc);
        } while (m);
    }
    wave_lds_sync();
}

struct InferArgs {
    const float *points;
    const void *diffuse;
    const void *specular;
    const float *density;
    const uint32_t *adjacency;
    const uint32_t *offsets;
    const uint2 *adj_diff;
    const float *rays;
    uint32_t num_rays;
    const uint32_t *start_point;
    uint32_t num_points; // a start cell at or past it: the ray takes no step
    const uint32_t *ray_perm;
    float thr, skip;
    uint32_t max_steps;
    uint16_t *rgba;
    uint32_t *stats;
    // tiled mode
    uint32_t num_images, H, W, th, tw;
    // q8
    float ds[3], dof[3], ss[3], sof[3];
    // camera renders: cameras of the images (device array); start cells per row
    const vt_camera *cams;
    uint32_t start_rows;
    // tiled and camera modes: launch order of the tiles (NULL = screen order)
    // and each tile's cost, written by the call (NULL = not recorded)
    const uint32_t *tile_order;
    uint32_t *tile_cost;
    // packed walk layout (vt_walk_layout), or wl_chunks = NULL to walk
    // adjacency / offsets / adj_diff
    const uint4 *wl_chunks;
    const uint2 *wl_links;
    const uint2 *wl_heads;
    const float4 *wl_cells;
    const uint16_t *wl_orig;
    // rays per start cell (0: one start cell per ray)
    uint32_t rays_per_start;
    // fp16 footprint tables (vt_quad_maps), or NULL to read the maps' texels
    const void *quad_d;
    const void *quad_s;
};

// MAP_CAMERA: tiled lanes whose rays come from cameras instead of a buffer.
// (Named constants: a kernel signature must not depend on an unnamed type,
// whose mangling differs between the host and the device compilation.)
constexpr int MAP_LINEAR = 0, MAP_TILED = 1, MAP_CAMERA = 2;

// Lane s of a launch renders ray slot_to_ray(s): tiled, lane s%64 of tile
// tile_of_slot(s) of the image batch (tile t in screen order is launch slot
// t, or the slot tile_order places it at); linear, ray s or ray_perm[s]
// (idle when that is not a ray index).
__device__ __forceinline__ uint32_t tile_of_slot(const InferArgs &a, uint32_t s)
{
    return a.tile_order ? a.tile_order[s >> 6] : s >> 6;
}

__device__ __forceinline__ uint32_t slot_to_ray(const InferArgs &a, uint32_t s, int map)
{
    if (map == MAP_TILED || map == MAP_CAMERA)
        return tiled_ray(tile_of_slot(a, s) * 64u + (s & 63u), a.num_images, a.H, a.W, a.th, a.tw);
    if (s >= a.num_rays)
        return NONE;
    if (!a.ray_perm)
        return s;
    const uint32_t r = a.ray_perm[s];
    return r < a.num_rays ? r : NONE;
}


template <int RD, int RS, bool Q8, bool STATS, int MAP, int CHUNK, bool PACKED, bool QUADS>
// 8 waves per SIMD need at most 64 VGPRs.  The fp16 kernel fits them; the q8
// kernel spills 12 bytes per lane and is still faster than at 7 waves
// (C4: 16.6 against 17.2 ms).  The statistics variants (tests and counters
// only) keep their larger register budget.
__global__ __launch_bounds__(INFER_BLOCK) __attribute__((amdgpu_waves_per_eu(STATS ? 1 : 8)))
void infer_kernel(InferArgs a, uint32_t total_slots)
{
    ShadeQueue &q = wave_queue();
    const int lane = (int)(threadIdx.x & 63u);
    // every lane stays in the wave's loop to the end (it shades for others)
    const uint32_t s = xcd_interleaved_block<INFER_XCD_CHUNK>() * blockDim.x + threadIdx.x;
    const uint32_t r = s < total_slots ? slot_to_ray(a, s, MAP) : NONE;
    bool active = r != NONE;
    using Tex = typename std::conditional<Q8, TexQ8<RD, RS, QUADS>, TexF16<RD, RS, QUADS>>::type;
    InferIntegrator<RD, RS, Tex> integ;
    integ.density = a.density;
    if constexpr (Q8) {
        integ.tex.diffuse = (const uint8_t *)(QUADS ? a.quad_d : a.diffuse);
        integ.tex.specular = (const uint8_t *)(QUADS ? a.quad_s : a.specular);
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            integ.tex.ds[c] = a.ds[c];
            integ.tex.dof[c] = a.dof[c];
            integ.tex.ss[c] = a.ss[c];
            integ.tex.sof[c] = a.sof[c];
        }
    } else {
        integ.tex.diffuse = (const uint2 *)(QUADS ? a.quad_d : a.diffuse);
        integ.tex.specular = (const uint2 *)(QUADS ? a.quad_s : a.specular);
    }
    integ.thr = a.thr;
    integ.skip = a.skip;
    integ.acc = mk(0.0f, 0.0f, 0.0f);
    integ.T = 1.0f;
    StatsAcc<STATS> st;
    st.begin(a.stats, r);
    typename std::conditional<PACKED, PackedWalk, WalkState>::type w;
    if (active) {
        uint32_t start;
        if constexpr (MAP == MAP_CAMERA) {
            // the ray of pixel (u, v) of image img, normalised as load_ray does
            const uint32_t hw = a.H * a.W, img = r / hw, rem = r - img * hw, v = rem / a.W, u = rem - v * a.W;
            f3 dd;
            camera_ray(a.cams[img], u, v, a.H, integ.o, dd);
            integ.d = divs(dd, __builtin_sqrtf(dot(dd, dd)));
            start = a.start_point[a.start_rows ? img * a.H + v : img];
        } else {
            load_ray(a.rays, r, integ.o, integ.d);
            start = a.start_point[a.rays_per_start ? r / a.rays_per_start : r];
        }
        float su, sv;
        oct_encode<RS>(mk(-integ.d.x, -integ.d.y, -integ.d.z), su, sv);
        Bilinear sb;
        if constexpr (QUADS) {
            sb = bilinear_quad<RS>(su, sv);
            q.si[lane] = (uint32_t)sb.i00;
        } else {
            sb = bilinear_setup<RS>(su, sv);
            q.si[lane] = (uint32_t)sb.i00 | (uint32_t)sb.i10 << 8 | (uint32_t)sb.i01 << 16 | (uint32_t)sb.i11 << 24;
        }
        q.sw[0][lane] = sb.w00;
        q.sw[1][lane] = sb.w10;
        q.sw[2][lane] = sb.w01;
        q.sw[3][lane] = sb.w11;
        if (start >= a.num_points) { // out of range: no step, rgba (0, 0, 0, 0)
            active = false;
            w.n = 0;
        } else if constexpr (PACKED) {
            walk_begin_packed(w, a.wl_heads, a.wl_cells, a.wl_chunks, start);
        } else {
            walk_begin(w, a.points, a.offsets, start);
        }
    }
    q.mask[lane] = 0ull;
    if (lane == 0)
        q.tail = 0;
    wave_lds_sync();
    uint32_t head = 0; // wave-uniform: entries shaded so far
    while (__ballot(active)) {
        if (active) {
            if constexpr (PACKED)
                // the q8 integrator reading the maps' texels leaves no register room for the preloaded
                // row; with its footprint tables it does (64 VGPRs, C4 11.76 -> 11.59 ms)
                active = walk_step_packed<!Q8 || QUADS>(w, integ.o, integ.d, a.wl_chunks, a.wl_links,
                                                        a.wl_cells, a.wl_orig, a.offsets, a.max_steps, integ, st);
            else
                active = walk_step<CHUNK>(w, integ.o, integ.d, a.points, a.adjacency, a.offsets, a.adj_diff,
                                          a.max_steps, integ, st);
        }
        wave_lds_sync();
        if (__builtin_amdgcn_readfirstlane(q.tail) - head >= 64u) {
            shade_batch<RD, RS>(q, head, 64, integ, lane);
            head += 64;
        }
    }
    const uint32_t rest = __builtin_amdgcn_readfirstlane(q.tail) - head;
    if (rest)
        shade_batch<RD, RS>(q, head, rest, integ, lane);
    if (MAP != MAP_LINEAR && a.tile_cost && s < total_slots) {
        // the tile's cost for the next launch's order: a wave takes about as
        // long as its longest walk and its most face records (every lane is
        // here: the wave loop has ended)
        const uint32_t nmax = wave_max_u32(r == NONE ? 0u : w.n);
        const uint32_t fmax = wave_max_u32(r == NONE ? 0u : st.face_count());
        if (lane == 0)
            a.tile_cost[tile_of_slot(a, s)] = tile_cost_of(nmax, fmax);
    }
    if (r == NONE)
        return;
    uint2 out;
    out.x = (uint32_t)f2h(integ.acc.x) | ((uint32_t)f2h(integ.acc.y) << 16);
    out.y = (uint32_t)f2h(integ.acc.z) | ((uint32_t)f2h(1.0f - integ.T) << 16);
    reinterpret_cast<uint2 *>(a.rgba)[r] = out;
    st.store(a.stats, r, w.n);
}

template <int RD, int RS, bool Q8, bool STATS, int MAP>
static int launch_one(const InferArgs &a, hipStream_t stream, uint32_t slots)
{
    uint32_t blocks = (slots + INFER_BLOCK - 1) / INFER_BLOCK;
    if (a.quad_d) {
        if (a.wl_chunks)
            infer_kernel<RD, RS, Q8, STATS, MAP, INFER_CHUNK, true, true><<<blocks, INFER_BLOCK, 0, stream>>>(a, slots);
        else
            infer_kernel<RD, RS, Q8, STATS, MAP, INFER_CHUNK, false, true><<<blocks, INFER_BLOCK, 0, stream>>>(a,
                                                                                                            slots);
        VT_LAUNCH_CHECK("infer_kernel");
        return VT_OK;
    }
    if (a.wl_chunks)
        infer_kernel<RD, RS, Q8, STATS, MAP, INFER_CHUNK, true, false><<<blocks, INFER_BLOCK, 0, stream>>>(a, slots);
    else
        infer_kernel<RD, RS, Q8, STATS, MAP, INFER_CHUNK, false, false><<<blocks, INFER_BLOCK, 0, stream>>>(a, slots);
    VT_LAUNCH_CHECK("infer_kernel");
    return VT_OK;
}

template <int RD, int RS, bool Q8>
static int launch_infer_rs(const InferArgs &a, bool stats, int map, hipStream_t stream, uint32_t lanes)
{
    if (map == MAP_CAMERA)
        return stats ? launch_one<RD, RS, Q8, true, MAP_CAMERA>(a, stream, lanes)
                     : launch_one<RD, RS, Q8, false, MAP_CAMERA>(a, stream, lanes);
    if (map == MAP_TILED)
        return stats ? launch_one<RD, RS, Q8, true, MAP_TILED>(a, stream, lanes)
                     : launch_one<RD, RS, Q8, false, MAP_TILED>(a, stream, lanes);
    return stats ? launch_one<RD, RS, Q8, true, MAP_LINEAR>(a, stream, lanes)
                 : launch_one<RD, RS, Q8, false, MAP_LINEAR>(a, stream, lanes);
}

template <bool Q8>
static int launch_infer(const InferArgs &a, uint32_t rd, uint32_t rs, bool stats, int map, hipStream_t stream,
                        uint32_t lanes)
{
    if (lanes == 0)
        return VT_OK;
    if (rd == 4 && rs == 4)
        return launch_infer_rs<4, 4, Q8>(a, stats, map, stream, lanes);
    if (rd == 8 && rs == 8)
        return launch_infer_rs<8, 8, Q8>(a, stats, map, stream, lanes);
    if (rd == 8 && rs == 4)
        return launch_infer_rs<8, 4, Q8>(a, stats, map, stream, lanes);
    if (rd == 4 && rs == 8)
        return launch_infer_rs<4, 8, Q8>(a, stats, map, stream, lanes);
    set_error("unsupported octahedral map resolution (diffuse %u, specular %u); compiled: 4, 8", rd, rs);
    return VT_ERR_UNSUPPORTED;
}

static int check_common(const void *points, const void *diffuse, const void *specular, const void *density,
                        const void *adjacency, const void *offsets, const void *adj_diff, const void *rays,
                        const void *start_point, const void *rgba)
{
    VT_REQUIRE(points && diffuse && specular && density && adjacency && offsets && adj_diff && rays &&
                   start_point && rgba,
               "null pointer argument");
    return VT_OK;
}

// The packed walk layout of a call, or the general walk when walk is NULL.
static int set_walk_layout(InferArgs &a, const vt_walk_layout *walk)
{
    if (!walk)
        return VT_OK;
    VT_REQUIRE(walk->chunks && walk->links && walk->heads && walk->cells && walk->orig,
               "null array in the walk layout");
    a.wl_chunks = reinterpret_cast<const uint4 *>(walk->chunks);
    a.wl_links = reinterpret_cast<const uint2 *>(walk->links);
    a.wl_heads = reinterpret_cast<const uint2 *>(walk->heads);
    a.wl_cells = reinterpret_cast<const float4 *>(walk->cells);
    a.wl_orig = walk->orig;
    return VT_OK;
}

// The footprint tables of a call, or the maps' texels when quads is NULL.
static int set_quad_maps(InferArgs &a, const vt_quad_maps *quads, uint32_t num_points, uint32_t diff_res,
                         uint32_t spec_res, uint32_t format)
{
    if (!quads)
        return VT_OK;
    VT_REQUIRE(quads->diffuse && quads->specular, "null table in the quad maps");
    VT_REQUIRE(quads->format == format, "quad maps of format %u (0 fp16, 1 q8) given to a %s render", quads->format,
               format == VT_QUAD_Q8 ? "q8" : "fp16");
    VT_REQUIRE(quads->num_points == num_points && quads->diff_res == diff_res && quads->spec_res == spec_res,
               "quad maps of %u cells at %u/%u texels per side, the render has %u cells at %u/%u",
               quads->num_points, quads->diff_res, quads->spec_res, num_points, diff_res, spec_res);
    a.quad_d = quads->diffuse;
    a.quad_s = quads->specular;
    return VT_OK;
}

} // namespace vt

using namespace vt;

extern "C" int vt_trace_infer_f16(const float *points, const uint16_t *diffuse, const uint16_t *specular,
                                  uint32_t diff_res, uint32_t spec_res, const float *density,
                                  const uint32_t *adjacency, const uint32_t *offsets, uint32_t num_points,
                                  const uint16_t *adj_diff, const float *rays, uint32_t num_rays,
                                  const uint32_t *start_point, const uint32_t *ray_perm, float weight_threshold,
                                  uint32_t max_intersections, float cell_skip_threshold, uint16_t *rgba,
                                  vt_ray_stats *stats, vt_stream_t stream)
{
    clear_error();
    if (num_rays == 0)
        return VT_OK;
    int rc = check_common(points, diffuse, specular, density, adjacency, offsets, adj_diff, rays, start_point, rgba);
    if (rc)
        return rc;
    InferArgs a{};
    a.num_points = num_points;
    a.points = points;
    a.diffuse = diffuse;
    a.specular = specular;
    a.density = density;
    a.adjacency = adjacency;
    a.offsets = offsets;
    a.adj_diff = reinterpret_cast<const uint2 *>(adj_diff);
    a.rays = rays;
    a.num_rays = num_rays;
    a.start_point = start_point;
    a.ray_perm = ray_perm;
    a.thr = weight_threshold;
    a.skip = cell_skip_threshold;
    a.max_steps = max_intersections;
    a.rgba = rgba;
    a.stats = reinterpret_cast<uint32_t *>(stats);
    return launch_infer<false>(a, diff_res, spec_res, stats != nullptr, MAP_LINEAR, as_stream(stream), num_rays);
}

extern "C" int vt_trace_infer_f16_tiled(const float *points, const uint16_t *diffuse, const uint16_t *specular,
                                        uint32_t diff_res, uint32_t spec_res, const float *density,
                                        const uint32_t *adjacency, const uint32_t *offsets, uint32_t num_points,
                                        const uint16_t *adj_diff, const float *rays, uint32_t num_images,
                                        uint32_t image_h, uint32_t image_w, uint32_t tile_h, uint32_t tile_w,
                                        const uint32_t *start_point, uint32_t rays_per_start,
                                        float weight_threshold,
                                        uint32_t max_intersections, float cell_skip_threshold, uint16_t *rgba,
                                        const uint32_t *tile_order, uint32_t *tile_cost,
                                        vt_ray_stats *stats, const vt_walk_layout *walk,
                                        const vt_quad_maps *quads, vt_stream_t stream)
{
    clear_error();
    if (num_images == 0 || image_h == 0 || image_w == 0)
        return VT_OK;
    int rc = check_common(points, diffuse, specular, density, adjacency, offsets, adj_diff, rays, start_point, rgba);
    if (rc)
        return rc;
    VT_REQUIRE(tile_h * tile_w == 64, "tile_h * tile_w must be 64 (one wave64 per tile), got %u x %u", tile_h,
               tile_w);
    uint64_t tiles = (uint64_t)((image_w + tile_w - 1) / tile_w) * ((image_h + tile_h - 1) / tile_h) * num_images;
    VT_REQUIRE(tiles * 64 < (1ull << 32), "image batch too large");
    VT_REQUIRE((uint64_t)num_images * image_h * image_w < (1ull << 32), "image batch too large");
    InferArgs a{};
    a.num_points = num_points;
    a.points = points;
    a.diffuse = diffuse;
    a.specular = specular;
    a.density = density;
    a.adjacency = adjacency;
    a.offsets = offsets;
    a.adj_diff = reinterpret_cast<const uint2 *>(adj_diff);
    a.rays = rays;
    a.num_rays = num_images * image_h * image_w;
    a.start_point = start_point;
    a.rays_per_start = rays_per_start;
    a.ray_perm = nullptr;
    a.thr = weight_threshold;
    a.skip = cell_skip_threshold;
    a.max_steps = max_intersections;
    a.rgba = rgba;
    a.stats = reinterpret_cast<uint32_t *>(stats);
    a.tile_order = tile_order;
    a.tile_cost = tile_cost;
    rc = set_walk_layout(a, walk);
    if (rc)
        return rc;
    rc = set_quad_maps(a, quads, num_points, diff_res, spec_res, VT_QUAD_F16);
    if (rc)
        return rc;
    a.num_images = num_images;
    a.H = image_h;
    a.W = image_w;
    a.th = tile_h;
    a.tw = tile_w;
    return launch_infer<false>(a, diff_res, spec_res, stats != nullptr, MAP_TILED, as_stream(stream),
                               (uint32_t)(tiles * 64));
}

extern "C" int vt_trace_infer_q8(const float *points, const uint8_t *diffuse, const uint8_t *specular,
                                 uint32_t diff_res, uint32_t spec_res, const float diff_scale[3],
                                 const float diff_offset[3], const float spec_scale[3], const float spec_offset[3],
                                 const float *density, const uint32_t *adjacency, const uint32_t *offsets,
                                 uint32_t num_points, const uint16_t *adj_diff, const float *rays,
                                 uint32_t num_rays, const uint32_t *start_point, const uint32_t *ray_perm,
                                 float weight_threshold, uint32_t max_intersections, float cell_skip_threshold,
                                 uint16_t *rgba, vt_ray_stats *stats, vt_stream_t stream)
{
    clear_error();
    if (num_rays == 0)
        return VT_OK;
    int rc = check_common(points, diffuse, specular, density, adjacency, offsets, adj_diff, rays, start_point, rgba);
    if (rc)
        return rc;
    VT_REQUIRE(diff_scale && diff_offset && spec_scale && spec_offset, "null dequantisation parameters");
    InferArgs a{};
    a.num_points = num_points;
    a.points = points;
    a.diffuse = diffuse;
    a.specular = specular;
    a.density = density;
    a.adjacency = adjacency;
    a.offsets = offsets;
    a.adj_diff = reinterpret_cast<const uint2 *>(adj_diff);
    a.rays = rays;
    a.num_rays = num_rays;
    a.start_point = start_point;
    a.ray_perm = ray_perm;
    a.thr = weight_threshold;
    a.skip = cell_skip_threshold;
    a.max_steps = max_intersections;
    a.rgba = rgba;
    a.stats = reinterpret_cast<uint32_t *>(stats);
    for (int c = 0; c < 3; ++c) {
        a.ds[c] = diff_scale[c];
        a.dof[c] = diff_offset[c];
        a.ss[c] = spec_scale[c];
        a.sof[c] = spec_offset[c];
    }
    return launch_infer<true>(a, diff_res, spec_res, stats != nullptr, MAP_LINEAR, as_stream(stream), num_rays);
}

extern "C" int vt_trace_infer_q8_tiled(const float *points, const uint8_t *diffuse, const uint8_t *specular,
                                       uint32_t diff_res, uint32_t spec_res, const float diff_scale[3],
                                       const float diff_offset[3], const float spec_scale[3],
                                       const float spec_offset[3], const float *density, const uint32_t *adjacency,
                                       const uint32_t *offsets, uint32_t num_points, const uint16_t *adj_diff,
                                       const float *rays, uint32_t num_images, uint32_t image_h, uint32_t image_w,
                                       uint32_t tile_h, uint32_t tile_w, const uint32_t *start_point,
                                       uint32_t rays_per_start, float weight_threshold, uint32_t max_intersections, float cell_skip_threshold,
                                       uint16_t *rgba, const uint32_t *tile_order, uint32_t *tile_cost,
                                       vt_ray_stats *stats, const vt_walk_layout *walk,
                                       const vt_quad_maps *quads, vt_stream_t stream)
{
    clear_error();
    if (num_images == 0 || image_h == 0 || image_w == 0)
        return VT_OK;
    int rc = check_common(points, diffuse, specular, density, adjacency, offsets, adj_diff, rays, start_point, rgba);
    if (rc)
        return rc;
    VT_REQUIRE(diff_scale && diff_offset && spec_scale && spec_offset, "null dequantisation parameters");
    VT_REQUIRE(tile_h * tile_w == 64, "tile_h * tile_w must be 64 (one wave64 per tile), got %u x %u", tile_h,
               tile_w);
    uint64_t tiles = (uint64_t)((image_w + tile_w - 1) / tile_w) * ((image_h + tile_h - 1) / tile_h) * num_images;
    VT_REQUIRE(tiles * 64 < (1ull << 32), "image batch too large");
    VT_REQUIRE((uint64_t)num_images * image_h * image_w < (1ull << 32), "image batch too large");
    InferArgs a{};
    a.num_points = num_points;
    a.points = points;
    a.diffuse = diffuse;
    a.specular = specular;
    a.density = density;
    a.adjacency = adjacency;
    a.offsets = offsets;
    a.adj_diff = reinterpret_cast<const uint2 *>(adj_diff);
    a.rays = rays;
    a.num_rays = num_images * image_h * image_w;
    a.start_point = start_point;
    a.rays_per_start = rays_per_start;
    a.thr = weight_threshold;
    a.skip = cell_skip_threshold;
    a.max_steps = max_intersections;
    a.rgba = rgba;
    a.stats = reinterpret_cast<uint32_t *>(stats);
    a.tile_order = tile_order;
    a.tile_cost = tile_cost;
    rc = set_walk_layout(a, walk);
    if (rc)
        return rc;
    rc = set_quad_maps(a, quads, num_points, diff_res, spec_res, VT_QUAD_Q8);
    if (rc)
        return rc;
    a.num_images = num_images;
    a.H = image_h;
    a.W = image_w;
    a.th = tile_h;
    a.tw = tile_w;
    for (int c = 0; c < 3; ++c) {
        a.ds[c] = diff_scale[c];
        a.dof[c] = diff_offset[c];
        a.ss[c] = spec_scale[c];
        a.sof[c] = spec_offset[c];
    }
    return launch_infer<true>(a, diff_res, spec_res, stats != nullptr, MAP_TILED, as_stream(stream),
                              (uint32_t)(tiles * 64));
}

namespace vt {

__global__ void camera_rays_kernel(const vt_camera *__restrict__ cams, uint32_t num_images, uint32_t H, uint32_t W,
                                   float *__restrict__ rays)
{
    const uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t hw = (uint64_t)H * W;
    if (r >= hw * num_images)
        return;
    const uint32_t img = (uint32_t)(r / hw), rem = (uint32_t)(r - img * hw), v = rem / W, u = rem - v * W;
    f3 o, d;
    camera_ray(cams[img], u, v, H, o, d);
    float *q = rays + 6 * r;
    q[0] = o.x;
    q[1] = o.y;
    q[2] = o.z;
    q[3] = d.x;
    q[4] = d.y;
    q[5] = d.z;
}

// Camera renders of num_images images (one launch).
template <bool Q8>
static int render_cameras(const InferArgs &a, const vt_camera *cameras, uint32_t num_images, int start_per_row,
                          uint32_t rd, uint32_t rs, bool stats, hipStream_t stream)
{
    VT_REQUIRE(a.th * a.tw == 64, "tile_h * tile_w must be 64 (one wave64 per tile), got %u x %u", a.th, a.tw);
    const uint64_t tiles = (uint64_t)((a.W + a.tw - 1) / a.tw) * ((a.H + a.th - 1) / a.th) * num_images;
    VT_REQUIRE(tiles * 64 < (1ull << 32) && (uint64_t)a.H * a.W * num_images < (1ull << 32), "image batch too large");
    InferArgs c = a;
    c.num_images = num_images;
    c.num_rays = num_images * a.H * a.W;
    c.cams = cameras;
    c.start_rows = start_per_row ? 1u : 0u;
    return launch_infer<Q8>(c, rd, rs, stats, MAP_CAMERA, stream, (uint32_t)(tiles * 64));
}

} // namespace vt

extern "C" int vt_camera_rays(const vt_camera *cameras, uint32_t num_images, uint32_t image_h, uint32_t image_w,
                              float *rays, vt_stream_t stream)
{
    clear_error();
    if (num_images == 0 || image_h == 0 || image_w == 0)
        return VT_OK;
    VT_REQUIRE(cameras && rays, "null pointer argument");
    const uint64_t total = (uint64_t)image_h * image_w * num_images;
    VT_REQUIRE(total < (1ull << 40), "image batch too large");
    camera_rays_kernel<<<(uint32_t)((total + 255) / 256), 256, 0, as_stream(stream)>>>(cameras, num_images, image_h,
                                                                                        image_w, rays);
    VT_LAUNCH_CHECK("camera_rays_kernel");
    return VT_OK;
}

extern "C" int vt_trace_infer_f16_camera(const float *points, const uint16_t *diffuse, const uint16_t *specular,
                                         uint32_t diff_res, uint32_t spec_res, const float *density,
                                         const uint32_t *adjacency, const uint32_t *offsets, uint32_t num_points,
                                         const uint16_t *adj_diff, const vt_camera *cameras, uint32_t num_images,
                                         uint32_t image_h, uint32_t image_w, uint32_t tile_h, uint32_t tile_w,
                                         const uint32_t *start_point, int start_per_row, float weight_threshold,
                                         uint32_t max_intersections, float cell_skip_threshold, uint16_t *rgba,
                                         const uint32_t *tile_order, uint32_t *tile_cost,
                                         vt_ray_stats *stats, const vt_walk_layout *walk,
                                         const vt_quad_maps *quads, vt_stream_t stream)
{
    clear_error();
    if (num_images == 0 || image_h == 0 || image_w == 0)
        return VT_OK;
    int rc = check_common(points, diffuse, specular, density, adjacency, offsets, adj_diff, cameras, start_point,
                          rgba);
    if (rc)
        return rc;
    InferArgs a{};
    a.num_points = num_points;
    a.points = points;
    a.diffuse = diffuse;
    a.specular = specular;
    a.density = density;
    a.adjacency = adjacency;
    a.offsets = offsets;
    a.adj_diff = reinterpret_cast<const uint2 *>(adj_diff);
    a.start_point = start_point;
    a.thr = weight_threshold;
    a.skip = cell_skip_threshold;
    a.max_steps = max_intersections;
    a.rgba = rgba;
    a.stats = reinterpret_cast<uint32_t *>(stats);
    a.tile_order = tile_order;
    a.tile_cost = tile_cost;
    rc = set_walk_layout(a, walk);
    if (rc)
        return rc;
    rc = set_quad_maps(a, quads, num_points, diff_res, spec_res, VT_QUAD_F16);
    if (rc)
        return rc;
    a.H = image_h;
    a.W = image_w;
    a.th = tile_h;
    a.tw = tile_w;
    return render_cameras<false>(a, cameras, num_images, start_per_row, diff_res, spec_res, stats != nullptr,
                                 as_stream(stream));
}

extern "C" int vt_trace_infer_q8_camera(const float *points, const uint8_t *diffuse, const uint8_t *specular,
                                        uint32_t diff_res, uint32_t spec_res, const float diff_scale[3],
                                        const float diff_offset[3], const float spec_scale[3],
                                        const float spec_offset[3], const float *density, const uint32_t *adjacency,
                                        const uint32_t *offsets, uint32_t num_points, const uint16_t *adj_diff,
                                        const vt_camera *cameras, uint32_t num_images, uint32_t image_h,
                                        uint32_t image_w, uint32_t tile_h, uint32_t tile_w,
                                        const uint32_t *start_point, int start_per_row, float weight_threshold,
                                        uint32_t max_intersections, float cell_skip_threshold, uint16_t *rgba,
                                        const uint32_t *tile_order, uint32_t *tile_cost,
                                        vt_ray_stats *stats, const vt_walk_layout *walk,
                                        const vt_quad_maps *quads, vt_stream_t stream)
{
    clear_error();
    if (num_images == 0 || image_h == 0 || image_w == 0)
        return VT_OK;
    int rc = check_common(points, diffuse, specular, density, adjacency, offsets, adj_diff, cameras, start_point,
                          rgba);
    if (rc)
        return rc;
    VT_REQUIRE(diff_scale && diff_offset && spec_scale && spec_offset, "null dequantisation parameters");
    InferArgs a{};
    a.num_points = num_points;
    a.points = points;
    a.diffuse = diffuse;
    a.specular = specular;
    a.density = density;
    a.adjacency = adjacency;
    a.offsets = offsets;
    a.adj_diff = reinterpret_cast<const uint2 *>(adj_diff);
    a.start_point = start_point;
    a.thr = weight_threshold;
    a.skip = cell_skip_threshold;
    a.max_steps = max_intersections;
    a.rgba = rgba;
    a.stats = reinterpret_cast<uint32_t *>(stats);
    a.tile_order = tile_order;
    a.tile_cost = tile_cost;
    rc = set_walk_layout(a, walk);
    if (rc)
        return rc;
    rc = set_quad_maps(a, quads, num_points, diff_res, spec_res, VT_QUAD_Q8);
    if (rc)
        return rc;
    a.H = image_h;
    a.W = image_w;
    a.th = tile_h;
    a.tw = tile_w;
    for (int c = 0; c < 3; ++c) {
        a.ds[c] = diff_scale[c];
        a.dof[c] = diff_offset[c];
        a.ss[c] = spec_scale[c];
        a.sof[c] = spec_offset[c];
    }
    return render_cameras<true>(a, cameras, num_images, start_per_row, diff_res, spec_res, stats != nullptr,
                                as_stream(stream));
}
