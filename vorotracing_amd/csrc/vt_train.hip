// vt_train.hip -- training traversal: forward (ray_integrator_octmap.cuh:57-282,
// kernel tracing_octmap.cu:151-230) and backward (ray_integrator_octmap.cuh:635-1027,
// kernel :232-340), with f32 or f16 attribute storage.
//
// Attribute maps are (num_points, 3*R*R), texel-major / channel-minor.  The
// backward scatters 28 gradient values per integrated cell (29 with
// point_error), lanes of one cell combined in LDS first, with global atomics
// (f32: hardware global_atomic_add_f32; f16: the packed-f16 global atomic
// add on the aligned pair holding the half, +0 into the other half).
#include <algorithm>
#include <type_traits>

#include "vt_internal.h"
#include "vt_walk.h"

namespace vt {

// ---------------------------------------------------------------------------
// attribute storage

template <typename A> struct Attr;

template <> struct Attr<float> {
    __device__ __forceinline__ static float load(const float *p, size_t i) { return p[i]; }
    __device__ __forceinline__ static void store(float *p, size_t i, float v) { p[i] = v; }
    __device__ __forceinline__ static void add(float *p, size_t i, float v) { atomicAdd(p + i, v); }
};

// f16 stored as raw 16-bit words
template <> struct Attr<uint16_t> {
    __device__ __forceinline__ static float load(const uint16_t *p, size_t i) { return h2f(p[i]); }
    __device__ __forceinline__ static void store(uint16_t *p, size_t i, float v) { p[i] = f2h(v); }
    // atomicAdd on a half (the reference's atomicAdd(__half*, __float2half(v))):
    // the hardware packed-f16 add on the aligned pair holding the half, with
    // +0 for the other half.  Each add rounds once to half.  The other half
    // is unchanged: x + (+0) = x for every x but -0, and gradient and
    // contribution buffers start at +0, which additions never turn into -0.
    // (A compare-and-swap loop on the 32-bit word took 70 times as long: the
    // lanes of a wave that add to one cell's texels serialise on its words.)
    // The global-address form: a flat atomic also counts against the LDS
    // wait counter, so the combining's LDS reads would wait for it.
    __device__ __forceinline__ static void add(uint16_t *p, size_t i, float v)
    {
        typedef _Float16 __attribute__((ext_vector_type(2))) half2_t;
        typedef __attribute__((address_space(1))) half2_t global_half2_t;
        const uintptr_t addr = reinterpret_cast<uintptr_t>(p + i);
        global_half2_t *pair = reinterpret_cast<global_half2_t *>(addr & ~(uintptr_t)3);
        const _Float16 h = __builtin_bit_cast(_Float16, f2h(v));
        const _Float16 z = __builtin_bit_cast(_Float16, (uint16_t)0);
        const half2_t val = (addr & 2) ? half2_t{z, h} : half2_t{h, z};
        (void)__builtin_amdgcn_global_atomic_fadd_v2f16(pair, val);
    }
    // Both halves of the 32-bit word at p + i (p + i 4-byte aligned): lo to
    // the half at p + i, hi to the one after it, in one packed add, each
    // half rounded once as by two separate adds.
    __device__ __forceinline__ static void add_pair(uint16_t *p, size_t i, float lo, float hi)
    {
        typedef _Float16 __attribute__((ext_vector_type(2))) half2_t;
        typedef __attribute__((address_space(1))) half2_t global_half2_t;
        global_half2_t *pair = reinterpret_cast<global_half2_t *>(reinterpret_cast<uintptr_t>(p + i));
        const half2_t val = {__builtin_bit_cast(_Float16, f2h(lo)), __builtin_bit_cast(_Float16, f2h(hi))};
        (void)__builtin_amdgcn_global_atomic_fadd_v2f16(pair, val);
    }
};

template <typename A, int RD, int RS> struct TrainTex {
    const A *__restrict__ diffuse;
    const A *__restrict__ specular;

    __device__ __forceinline__ static f3 sample(const A *__restrict__ m, const Bilinear &b)
    {
        float v[3];
#pragma unroll
        for (int c = 0; c < 3; ++c)
            v[c] = bil_mix(b, Attr<A>::load(m, b.i00 * 3 + c), Attr<A>::load(m, b.i10 * 3 + c),
                           Attr<A>::load(m, b.i01 * 3 + c), Attr<A>::load(m, b.i11 * 3 + c));
        return mk(v[0], v[1], v[2]);
    }
    // sigmoid(diffuse(probe) + specular(spec taps)); diffuse taps out in db
    __device__ __forceinline__ f3 color(uint32_t cell, f3 o, f3 d, float t0, f3 p, const Bilinear &spec,
                                        Bilinear &db) const
    {
        f3 pd = probe_dir(o, d, t0, p);
        float u, v;
        oct_encode<RD>(pd, u, v);
        db = bilinear_setup<RD>(u, v);
        f3 a = sample(diffuse + (size_t)cell * (3 * RD * RD), db);
        f3 b = sample(specular + (size_t)cell * (3 * RS * RS), spec);
        f3 lg = add(a, b);
        return mk(sigmoid(lg.x), sigmoid(lg.y), sigmoid(lg.z));
    }
};

// ---------------------------------------------------------------------------
// Same-cell combining of scatters.  Rays of one wave often integrate the same
// cell in the same step (all rays of a camera share the start cell and its
// neighbours), and hardware atomics to one address serialise.  A scatter
// therefore groups the active lanes by cell, leader by leader (the lowest
// pending lane).  The forward's contribution sums a group's weights with
// v_readlane (FwdIntegrator::scatter_contribution); the backward's records
// go through a per-wave LDS row table (BwdIntegrator::scatter).  Only the
// order of the floating-point additions changes (atomics have no defined
// order anyway).

constexpr int TRAIN_BLOCK = 64; // one wave per block: each wave's LDS is freed when it ends
// waves per SIMD the training kernels' register budgets allow (the
// forward spills 20 bytes at 6; the backward keeps 112 VGPRs at 4)
constexpr uint32_t TRAIN_FWD_WAVES = 6, TRAIN_BWD_WAVES = 4;
constexpr int TRAIN_WAVES = TRAIN_BLOCK / 64;
constexpr int TRAIN_CHUNK = 8;      // face records read together per exit-face step (forward)
constexpr int TRAIN_BWD_CHUNK = 12; // the same in the backward (C2: 3.93-3.98 against 4.04-4.07 ms with 8;
                                    // the forward is faster with 8 at C5)
constexpr uint32_t TRAIN_XCD_CHUNK = 32; // blocks per XCD turn (xcd_interleaved_block)

// The backward's scatter record of one lane: 12 diffuse and 12 specular
// values (tap-major, 3 channels each), dL/ds, the point_error term and the
// point gradient, then the diffuse and specular tap words (words 29, 30).
// Each scattering lane writes its record as one row of the wave's LDS table;
// ROW_STRIDE keeps rows 16-byte aligned and puts 8 consecutive lanes'
// 16-byte stores on distinct banks.  Row 64 stays zero and is read in place
// of absent group members.
constexpr int REC_COLS = 29;
constexpr int REC_DTAPS = 29, REC_STAPS = 30;
constexpr int ROW_STRIDE = 36;
constexpr int ROW_TABLE_FLOATS = 65 * ROW_STRIDE;

// Ray of lane slot s: perm[s] when a lane order is given (entries past
// num_rays leave the lane idle), else 8x8 screen tiles of row-major images,
// or ray order.
constexpr uint32_t TRAIN_TILE = 8;
// Tile strips of the training kernels, 2 tiles wide (C2: forward 1.13-1.15
// against 1.15-1.18 ms, backward 3.98-4.03 against 4.04-4.09 with strips of
// 4, which inference keeps).
#ifndef VT_TRAIN_TILE_STRIP
#define VT_TRAIN_TILE_STRIP 2
#endif
constexpr uint32_t TRAIN_TILE_STRIP = VT_TRAIN_TILE_STRIP;

// Tiles of a training launch: the screen tiles of image lanes, or the waves
// of 64 consecutive ray_perm entries of a sorted flat batch; 0 for rays in
// batch order.
__host__ __device__ inline uint32_t train_tiles(uint32_t num_rays, bool perm, uint32_t ni, uint32_t h, uint32_t w)
{
    if (perm)
        return (num_rays + 63u) / 64u;
    return ni * ((w + TRAIN_TILE - 1) / TRAIN_TILE) * ((h + TRAIN_TILE - 1) / TRAIN_TILE);
}

// Slot s of a tiled training launch: the tile its wave runs (NONE past the
// last), the lane's ray within the tile's 64 (NONE for the idle lanes of a
// half-wave) and whether the wave runs half a tile.  With a tile order,
// wave j runs tile tile_order[j], except that the first k tiles of the
// order, k = tile_order[tiles] clamped to the waves the launch added for
// them, run as two half-waves each: waves 2i and 2i + 1 take the first and
// the last 32 rays of tile tile_order[i] (rows 0-3 and 4-7 of a screen
// tile) on lanes 0-31, and wave 2k + j takes tile tile_order[k + j].  A long
// tile, which the launch would otherwise end waiting for, then ends about as
// early as the rest.  The forward (ORDER_ONLY_TO_SPLIT) keeps its own order
// when k is 0: an order alone made it slower.
struct TrainSlot {
    uint32_t tile, within;
    bool half;
};

template <bool ORDER_ONLY_TO_SPLIT>
__device__ __forceinline__ TrainSlot train_slot(uint32_t s, uint32_t tiles, const uint32_t *tile_order)
{
    TrainSlot r{s >> 6, s & 63u, false};
    if (!tile_order) {
        if (r.tile >= tiles)
            r.tile = NONE;
        return r;
    }
    const uint32_t waves = gridDim.x * (blockDim.x / 64u);
    const uint32_t extra = waves > tiles ? waves - tiles : 0u;
    const uint32_t k = min(min(tile_order[tiles], tiles), extra);
    if (ORDER_ONLY_TO_SPLIT && k == 0) {
        if (r.tile >= tiles)
            r.tile = NONE;
        return r;
    }
    uint32_t t = r.tile;
    if (t < 2u * k) {
        r.half = true;
        r.within = r.within < 32u ? r.within + (t & 1u) * 32u : NONE;
        t >>= 1;
    } else {
        t -= k;
    }
    r.tile = t < tiles ? tile_order[t] : NONE;
    return r;
}

template <bool ORDER_ONLY_TO_SPLIT>
__device__ __forceinline__ uint32_t train_ray(uint32_t s, uint32_t num_rays, const uint32_t *perm, uint32_t ni,
                                              uint32_t h, uint32_t w, const uint32_t *tile_order)
{
    if (perm) {
        uint32_t q = s;
        if (tile_order) {
            const TrainSlot t = train_slot<ORDER_ONLY_TO_SPLIT>(s, train_tiles(num_rays, true, 0, 0, 0), tile_order);
            if (t.tile == NONE || t.within == NONE)
                return NONE;
            q = t.tile * 64u + t.within;
        }
        if (q >= num_rays)
            return NONE;
        const uint32_t r = perm[q];
        return r < num_rays ? r : NONE;
    }
    if (ni) {
        const TrainSlot t = train_slot<ORDER_ONLY_TO_SPLIT>(s, train_tiles(num_rays, false, ni, h, w), tile_order);
        if (t.tile == NONE || t.within == NONE)
            return NONE;
        return tiled_ray<TRAIN_TILE_STRIP>(t.tile * 64u + t.within, ni, h, w, TRAIN_TILE, TRAIN_TILE);
    }
    return s < num_rays ? s : NONE;
}

// ---------------------------------------------------------------------------
// forward

struct FwdArgs {
    const float *points;
    const void *diffuse, *specular;
    const float *density;
    const uint32_t *adjacency, *offsets;
    const uint2 *adj_diff;
    const float *rays;
    uint32_t num_rays;
    const uint32_t *ray_perm;          // lane order, or null
    uint32_t num_images, img_h, img_w; // tiled lane order when num_images > 0 and no ray_perm
    const uint32_t *start_point;
    uint32_t num_points; // a start cell at or past it: the ray takes no step
    uint32_t K;
    const float *quantiles;
    float thr;
    uint32_t max_steps;
    void *rgba;
    float *depth;
    uint32_t *depth_idx;
    void *contribution;
    uint32_t *n_out;
    float *distortion, *W_total, *S_total, *t_far;
    uint32_t *stats;
    const uint32_t *tile_order; // tiled lane order: launch order of the tiles, or null (screen order)
    uint32_t *tile_cost;        // tiled lane order: each tile's cost (tile_cost_of), or null
};

// RayIntegratorOctMap::integrate_cell (ray_integrator_octmap.cuh:102-152)
template <typename A, int RD, int RS> struct FwdIntegrator {
    f3 o, d;
    const float *__restrict__ density;
    TrainTex<A, RD, RS> tex;
    Bilinear spec;
    float thr;
    A *contribution;
    const float *qthr;
    uint32_t nq, qi;
    float qval;
    float *qdepth;
    uint32_t *qidx;
    f3 acc;
    float T, W, S, D, self, tfar;

    // contribution[cell] += w.  The lanes of one cell are summed first, in
    // lane order, for the group's lowest lane (v_readlane over the members:
    // scalar work, no LDS), and the groups' sums then leave in one atomic
    // instruction.
    __device__ __forceinline__ void scatter_contribution(uint32_t cell, float w)
    {
        const int lane = (int)(threadIdx.x & 63u);
        uint64_t pend = __ballot(1);
        float mine = 0.0f;
        bool leader = false;
        while (pend) {
            const int ll = (int)__builtin_ctzll(pend);
            const uint32_t lead = __builtin_amdgcn_readlane(cell, ll);
            uint64_t m = __ballot(cell == lead) & pend;
            pend &= ~m;
            float sum = 0.0f;
            do {
                const int src = (int)__builtin_ctzll(m);
                m &= m - 1;
                sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), src));
            } while (m);
            if (lane == ll) {
                mine = sum;
                leader = true;
            }
        }
        if (leader && mine != 0.0f) // weights are >= 0: a zero sum adds nothing
            Attr<A>::add(contribution, cell, mine);
    }

    float pdens; // density of the current cell, loaded by begin_cell

    __device__ __forceinline__ void begin_cell(uint32_t cell) { pdens = density[cell]; }

    template <class St>
    __device__ __forceinline__ bool integrate(uint32_t cell, float t0, float t1, f3 p, f3, St &st)
    {
        float sig = pdens;
        f3 rgb = mk(0.0f, 0.0f, 0.0f);
        if (sig > 1e-6f) {
            st.shade();
            Bilinear db;
            rgb = tex.color(cell, o, d, t0, p, spec, db);
        }
        float dt = __builtin_fmaxf(t1 - t0, 0.0f);
        float alpha = 1.0f - vt_expf(-sig * dt);
        float w = T * alpha;

        float s0 = 1.0f - 1.0f / (1.0f + t0);
        float s1 = 1.0f - 1.0f / (1.0f + t1);
        float mid = 0.5f * (s0 + s1);
        float ds = s1 - s0;
        D = fma_(w, fma_(mid, W, -S), D);
        self = fma_(w * w, ds, self);
        W = W + w;
        S = fma_(w, mid, S);
        if (t1 > tfar)
            tfar = t1;

        if (contribution)
            scatter_contribution(cell, w);
        acc = vfma(w, rgb, acc);

        float nextT = T * (1.0f - alpha);
        while (qi < nq && nextT < qval) {
            qdepth[qi] = t0 + vt_logf(T / qval) / sig;
            qidx[qi] = cell;
            qi++;
            if (qi < nq)
                qval = qthr[qi];
        }
        T = nextT;
        return T > thr;
    }
};

// 6 waves per SIMD (80 VGPRs, 20 bytes spilled) beat the 5 that the
// unspilled kernel allows (1.13-1.16 against 1.19-1.21 ms at C2): more waves
// hide more of the walk's load latency.
// The forward of ray r; returns the walk's step count, and in faces the face
// records it searched.
template <typename A, int RD, int RS, bool STATS>
__device__ __forceinline__ uint32_t fwd_ray(const FwdArgs &a, uint32_t r, uint32_t &faces)
{
    FwdIntegrator<A, RD, RS> it;
    load_ray(a.rays, r, it.o, it.d);
    it.density = a.density;
    it.tex.diffuse = (const A *)a.diffuse;
    it.tex.specular = (const A *)a.specular;
    float su, sv;
    oct_encode<RS>(mk(-it.d.x, -it.d.y, -it.d.z), su, sv);
    it.spec = bilinear_setup<RS>(su, sv);
    it.thr = a.thr;
    it.contribution = (A *)a.contribution;
    uint32_t K = a.quantiles ? a.K : 0;
    it.nq = K;
    it.qi = 0;
    it.qthr = K ? a.quantiles + (size_t)r * K : nullptr;
    it.qval = K ? it.qthr[0] : 0.0f;
    it.qdepth = K ? a.depth + (size_t)r * K : nullptr;
    it.qidx = K ? a.depth_idx + (size_t)r * K : nullptr;
    it.acc = mk(0.0f, 0.0f, 0.0f);
    it.T = 1.0f;
    it.W = it.S = it.D = it.self = it.tfar = 0.0f;
    StatsAcc<STATS> st;
    st.begin(a.stats, r);
    const uint32_t start = a.start_point[r];
    const uint32_t n = start < a.num_points ? walk<TRAIN_CHUNK>(it.o, it.d, a.points, a.adjacency, a.offsets,
                                                                a.adj_diff, start, a.max_steps, it, st)
                                            : 0u;
    for (uint32_t i = it.qi; i < K; ++i) {
        a.depth[(size_t)r * K + i] = -1.0f;
        a.depth_idx[(size_t)r * K + i] = NONE;
    }
    A *rgba = (A *)a.rgba;
    Attr<A>::store(rgba, 4 * (size_t)r + 0, it.acc.x);
    Attr<A>::store(rgba, 4 * (size_t)r + 1, it.acc.y);
    Attr<A>::store(rgba, 4 * (size_t)r + 2, it.acc.z);
    Attr<A>::store(rgba, 4 * (size_t)r + 3, 1.0f - it.T);
    if (a.n_out)
        a.n_out[r] = n;
    a.distortion[r] = fma_(2.0f, it.D, it.self / 3.0f);
    a.W_total[r] = it.W;
    a.S_total[r] = it.S;
    a.t_far[r] = it.tfar;
    st.store(a.stats, r, n);
    faces = st.face_count();
    return n;
}

template <typename A, int RD, int RS, bool STATS>
__global__ __launch_bounds__(TRAIN_BLOCK) __attribute__((amdgpu_waves_per_eu(TRAIN_FWD_WAVES)))
void fwd_kernel(FwdArgs a)
{
    const uint32_t s = xcd_interleaved_block<TRAIN_XCD_CHUNK>() * blockDim.x + threadIdx.x;
    const uint32_t r = train_ray<true>(s, a.num_rays, a.ray_perm, a.num_images, a.img_h, a.img_w, a.tile_order);
    uint32_t n = 0, faces = 0;
    if (r != NONE)
        n = fwd_ray<A, RD, RS, STATS>(a, r, faces);
    if (a.tile_cost && (a.num_images || a.ray_perm)) {
        // tiled launches are whole waves, and every lane is here; a split
        // tile records the larger of its halves' costs (the slower half is
        // what bounds it), in an atomic max (the caller cleared the costs
        // before an ordered launch)
        const uint32_t nmax = wave_max_u32(n), fmax = wave_max_u32(faces);
        if ((threadIdx.x & 63u) == 0) {
            const TrainSlot t = train_slot<true>(
                s, train_tiles(a.num_rays, a.ray_perm != nullptr, a.num_images, a.img_h, a.img_w), a.tile_order);
            if (t.tile != NONE) {
                if (t.half)
                    atomicMax(a.tile_cost + t.tile, tile_cost_of(nmax, fmax));
                else
                    a.tile_cost[t.tile] = tile_cost_of(nmax, fmax);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// backward

struct BwdArgs {
    const float *points;
    const void *diffuse, *specular;
    const float *density;
    const uint32_t *adjacency, *offsets;
    const uint2 *adj_diff;
    const float *rays;
    uint32_t num_rays;
    const uint32_t *ray_perm;          // lane order, or null
    uint32_t num_images, img_h, img_w; // tiled lane order when num_images > 0 and no ray_perm
    const uint32_t *start_point;
    uint32_t num_points; // a start cell at or past it: the ray takes no step
    const void *rgba, *rgba_grad;
    uint32_t K;
    const float *quantiles;
    const uint32_t *depth_idx;
    const float *depth_grad;
    const void *ray_error;
    float contribution_alpha_grad;
    const float *distortion, *distortion_grad, *W_total, *S_total;
    float thr;
    uint32_t max_steps;
    float *cell_grad; // (num_points, 4): point gradient, density gradient
    void *diffuse_grad, *specular_grad;
    void *point_error;
    uint32_t *stats;
    const uint32_t *tile_order; // tiled lane order: launch order of the tiles, or null (screen order)
};

// ray_integrator.cuh:39-53
__device__ __forceinline__ f3 cell_intersection_grad(f3 prim, f3 opp, f3 o, f3 d)
{
    f3 fo = mk((prim.x + opp.x) * 0.5f, (prim.y + opp.y) * 0.5f, (prim.z + opp.z) * 0.5f);
    f3 n = sub(opp, prim);
    float num = dot(sub(fo, o), n);
    float dp = dot(n, d);
    f3 op = sub(o, prim);
    f3 g = mk(fma_(num, d.x, dp * op.x), fma_(num, d.y, dp * op.y), fma_(num, d.z, dp * op.z));
    return divs(g, dp * dp);
}

// RayIntegratorOctMapBackward::integrate_cell (ray_integrator_octmap.cuh:683-860)
template <typename A, int RD, int RS> struct BwdIntegrator {
    f3 o, d;
    const float *__restrict__ density;
    TrainTex<A, RD, RS> tex;
    Bilinear spec;
    float thr;
    f3 acc;
    float T;
    float cur_depth_grad;
    uint32_t qi, nq;
    float qval;
    const float *qthr, *depth_grad;
    float *cell_grad; // per cell (point gradient x, y, z, density gradient)
    A *diffuse_grad, *specular_grad, *point_error;
    f3 prev_geom, prev_grad, cur_grad, next_grad;
    uint32_t prev_idx;
    f3 fwd_rgb, fwd_rgb_grad;
    float fwd_alpha, fwd_alpha_grad, ray_error;
    float W_run, S_run, W_total, S_total, dist_grad, D_total, D_running;
    float *rows;        // this wave's LDS row table, ROW_TABLE_FLOATS floats
    uint32_t spec_taps; // the ray's four specular taps, 8 bits each

    static constexpr int ND = 3 * RD * RD, NS = 3 * RS * RS;

    // The texture, density and point_error gradients of an integrated cell
    // are held until the walk has integrated the next cell (or ends): the
    // cell's point gradient is then complete, and both go out in one scatter
    // keyed by the cell, so that one combining pass serves both.  Held: the
    // four diffuse taps (texel indices < 256, 8 bits each; HELD_NO_COLOR when
    // the cell was not shaded) with their weights, the logit gradient, dL/ds
    // and the point_error term.
    static constexpr uint32_t HELD_NO_COLOR = 0xffffffffu;
    uint32_t held_taps;
    float held_w[4], held_gl[3], held_ds, held_perr;

    __device__ __forceinline__ void hold(bool has_color, const Bilinear &db, const float *gl, float dL_ds, float perr)
    {
        static_assert(RD * RD <= 256, "diffuse tap indices are packed in 8 bits");
        held_taps = HELD_NO_COLOR;
        if (has_color) { // db is set only for shaded cells
            held_taps = (uint32_t)db.i00 | (uint32_t)db.i10 << 8 | (uint32_t)db.i01 << 16 | (uint32_t)db.i11 << 24;
            held_w[0] = db.w00;
            held_w[1] = db.w10;
            held_w[2] = db.w01;
            held_w[3] = db.w11;
        }
        held_gl[0] = gl[0];
        held_gl[1] = gl[1];
        held_gl[2] = gl[2];
        held_ds = dL_ds;
        held_perr = perr;
    }

    // What a lane needs to send column k of a combined record (k in
    // [0, REC_COLS)): the tap it reads (a byte of the diffuse or specular tap
    // word; none for the other columns) and the target, element
    // cell * stride + 3 * tap + off of base.  Set once per scatter, not per
    // group.  A texture column of an unshaded cell (taps unset) and the
    // point_error column without that output send nothing.
    struct Column {
        uint32_t k, sh, tmask;
        bool diffuse_taps, on;
        bool attr; // the target holds attribute values (textures, point_error), else f32
        void *base;
        uint32_t stride, off, taps; // taps: texels of the map (1 for other columns)
    };

    __device__ __forceinline__ Column column(uint32_t k) const
    {
        Column c;
        const uint32_t kt = k < 12u ? k : k - 12u;
        c.k = k;
        c.sh = k < 24u ? 8u * (kt / 3u) : 0u;
        c.tmask = k < 24u ? 0xffu : 0u;
        c.diffuse_taps = k < 12u;
        c.on = k != 25u || point_error;
        c.taps = k < 12u ? RD * RD : k < 24u ? RS * RS : 1u;
        c.attr = k < 24u || k == 25u;
        c.base = k < 12u    ? static_cast<void *>(diffuse_grad)
                 : k < 24u  ? static_cast<void *>(specular_grad)
                 : k == 25u ? static_cast<void *>(point_error)
                            : static_cast<void *>(cell_grad);
        c.stride = k < 12u ? (uint32_t)ND : k < 24u ? (uint32_t)NS : k == 25u ? 1u : 4u;
        c.off = k < 24u ? kt - 3u * (kt / 3u) : k == 24u ? 3u : k == 25u ? 0u : k - 26u;
        return c;
    }

    // One add of a combined column: one atomic instruction for every target
    // (f32), or one per storage type (f16 attributes, f32 slots).
    __device__ __forceinline__ void column_send(const Column &c, uint32_t cell, uint32_t tap, float x)
    {
        if (c.on && tap < c.taps) {
            const size_t i = (size_t)cell * c.stride + 3u * tap + c.off;
            if (std::is_same<A, float>::value || !c.attr) {
                atomicAdd(static_cast<float *>(c.base) + i, x);
            } else {
                // halves of one 32-bit word in separate instructions: lanes
                // adding to the same word in one atomic instruction serialise
#pragma unroll 1
                for (uint32_t half = 0; half < 2; ++half)
                    if ((i & 1) == half)
                        Attr<A>::add(static_cast<A *>(c.base), i, x);
            }
        }
    }

    // The sends of one combining pass.  Every lane of the pass calls it
    // (a converged region), and a lane's column is the next one after the
    // column of the lane below it in the pass.  f32: one atomic per lane.
    // f16 attributes: the two halves of a 32-bit word usually belong to a
    // column and the next one (a tap's channels, or one tap's last channel
    // and the next tap's first); the lane of the first then adds both in one
    // packed atomic and the next lane skips, and every other lane adds its
    // half alone, all in one instruction (lanes that add to one word in one
    // instruction serialise; here no two do unless a wrapped tap repeats a
    // texel).  Each value is still added exactly once.
    __device__ __forceinline__ void column_send_pass(const Column &c, uint32_t cell, uint32_t tap, float x,
                                                     uint32_t lane)
    {
        const bool send = x != 0.0f && c.on && tap < c.taps;
        const size_t i = (size_t)cell * c.stride + 3u * tap + c.off;
        if constexpr (std::is_same<A, float>::value) {
            if (send)
                atomicAdd(static_cast<float *>(c.base) + i, x);
        } else {
            if (!c.attr) {
                if (send)
                    atomicAdd(static_cast<float *>(c.base) + i, x);
                return;
            }
            column_send_f16(c, i, x, send, lane);
        }
    }

    __device__ __forceinline__ void column_send_f16(const Column &c, size_t i, float x, bool send, uint32_t lane)
    {
        const uint64_t here = __ballot(1);
        const uint64_t above = lane < 63u ? here & (~0ull << (lane + 1u)) : 0ull;
        const uint64_t below = here & ((1ull << lane) - 1ull);
        const uint32_t next = above ? (uint32_t)__builtin_ctzll(above) : lane;
        // a texture column and the next column of the same map
        const bool pairs_up = c.k < 24u && c.k != 11u && c.k != 23u;
        const uint32_t a_lo = (uint32_t)reinterpret_cast<uintptr_t>(static_cast<A *>(c.base) + i);
        const uint64_t sending = __ballot(send && c.k < 24u);
        const uint32_t a_next = __shfl(a_lo, (int)next, 64);
        const float x_next = __shfl(x, (int)next, 64);
        const bool owner = send && pairs_up && above && ((sending >> next) & 1u) && (a_lo & 3u) == 0 &&
                           a_next == a_lo + 2u;
        const uint64_t owners = __ballot(owner);
        const bool taken = below && ((owners >> (63 - __builtin_clzll(below))) & 1u);
        if (owner)
            Attr<A>::add_pair(static_cast<A *>(c.base), i, x, x_next);
        else if (send && !taken)
            Attr<A>::add(static_cast<A *>(c.base), i, x);
    }

    // Sum of column c (column k of the row table) over the members `mem` of
    // one cell's group (ll: the lowest member; uniform: every member has the
    // leader's taps).  acc is the sum for tap t0, the leader's; when taps
    // differ, acc1 is the sum for one other tap t1, and a third tap sends
    // acc1 and takes its place.
    __device__ __forceinline__ void column_sum(const Column &c, uint32_t k, uint32_t lead, uint64_t mem, int ll,
                                               bool uniform, uint32_t t0, float &acc, uint32_t &t1, float &acc1)
    {
        const float *col = rows + k;
        uint64_t m = mem;
        if (uniform) {
            if ((mem & (mem - 1)) == 0) { // a lone lane: its own row
                acc = col[ll * ROW_STRIDE];
                return;
            }
            do { // four members per pass; the zero row stands in for absent ones
                const int s0 = (int)__builtin_ctzll(m);
                m &= m - 1;
                const int s1 = m ? (int)__builtin_ctzll(m) : 64;
                m &= m - 1;
                const int s2 = m ? (int)__builtin_ctzll(m) : 64;
                m &= m - 1;
                const int s3 = m ? (int)__builtin_ctzll(m) : 64;
                m &= m - 1;
                const float x0 = col[s0 * ROW_STRIDE], x1 = col[s1 * ROW_STRIDE];
                const float x2 = col[s2 * ROW_STRIDE], x3 = col[s3 * ROW_STRIDE];
                acc += (x0 + x1) + (x2 + x3);
            } while (m);
            return;
        }
        const float *tw = rows + (c.diffuse_taps ? REC_DTAPS : REC_STAPS);
        do {
            int sm[4];
            float x[4];
            uint32_t w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sm[j] = m ? (int)__builtin_ctzll(m) : 64;
                m &= m - 1;
                x[j] = col[sm[j] * ROW_STRIDE];
                w[j] = __float_as_uint(tw[sm[j] * ROW_STRIDE]);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (sm[j] == 64)
                    break; // no more members (wave-uniform)
                const uint32_t tap = (w[j] >> c.sh) & c.tmask;
                const bool in0 = tap == t0, in1 = tap == t1;
                acc += in0 ? x[j] : 0.0f;
                acc1 += in1 ? x[j] : 0.0f;
                if (!in0 && !in1) {
                    if (acc1 != 0.0f)
                        column_send(c, lead, t1, acc1);
                    t1 = tap;
                    acc1 = x[j];
                }
            }
        } while (m);
    }

    // The combining passes of one scatter; ONE: every column has its own
    // lane (at least REC_COLS lanes scatter), so the column is set up once;
    // otherwise a lane takes several columns.  With at least 2 * REC_COLS
    // lanes, groups of a single lane are set aside and sent two per pass
    // afterwards: lanes of rank k < REC_COLS send column k of the first,
    // lanes of rank REC_COLS + k column k of the second.
    template <bool ONE>
    __device__ __forceinline__ void combine(uint32_t cell, uint64_t act, uint32_t nact, uint32_t arank, uint32_t lane)
    {
        const bool pair = ONE && nact >= 2u * (uint32_t)REC_COLS;
        const uint32_t half = arank >= (uint32_t)REC_COLS ? 1u : 0u;
        Column c1;
        if (ONE)
            c1 = column(arank - half * (uint32_t)REC_COLS);
        uint64_t pend = act, singles = 0;
        while (pend) { // one group per pass, at most 64
            const int ll = (int)__builtin_ctzll(pend);
            const uint32_t lead = __builtin_amdgcn_readlane(cell, ll);
            const uint64_t mem = __ballot(cell == lead) & pend;
            pend &= ~mem;
            if (pair && (mem & (mem - 1)) == 0) {
                singles |= mem;
                continue;
            }
            const uint32_t ldt = __builtin_amdgcn_readlane(held_taps, ll);
            const uint32_t lst = __builtin_amdgcn_readlane(spec_taps, ll);
            // do all members share the leader's taps? (the usual case)
            const bool uniform =
                (mem & (mem - 1)) == 0 || __ballot(((mem >> lane) & 1u) && (held_taps != ldt || spec_taps != lst)) == 0;
            for (uint32_t k = arank; k < (uint32_t)REC_COLS; k += nact) {
                const Column c = ONE ? c1 : column(k);
                const uint32_t t0 = ((c.diffuse_taps ? ldt : lst) >> c.sh) & c.tmask;
                uint32_t t1 = 0xffffffffu;
                float acc = 0.0f, acc1 = 0.0f;
                column_sum(c, k, lead, mem, ll, uniform, t0, acc, t1, acc1);
                column_send_pass(c, lead, t0, acc, lane);
                if (__ballot(acc1 != 0.0f)) // second sums: only where some member's taps differ
                    column_send_pass(c, lead, t1, acc1, lane);
            }
        }
        while (singles) { // (pair only) two lone lanes per pass
            const int la = (int)__builtin_ctzll(singles);
            singles &= singles - 1;
            const int lb = singles ? (int)__builtin_ctzll(singles) : 64;
            singles &= singles - 1;
            const uint32_t ca = __builtin_amdgcn_readlane(cell, la), cb = __builtin_amdgcn_readlane(cell, lb & 63);
            const uint32_t da = __builtin_amdgcn_readlane(held_taps, la), db = __builtin_amdgcn_readlane(held_taps, lb & 63);
            const uint32_t sa = __builtin_amdgcn_readlane(spec_taps, la), sb = __builtin_amdgcn_readlane(spec_taps, lb & 63);
            const int mine = half ? lb : la;
            if (arank < 2u * (uint32_t)REC_COLS && mine < 64) {
                const float x = rows[mine * ROW_STRIDE + (c1.k)];
                const uint32_t t = (((c1.diffuse_taps ? (half ? db : da) : (half ? sb : sa))) >> c1.sh) & c1.tmask;
                column_send_pass(c1, half ? cb : ca, t, x, lane);
            }
        }
    }

    // Scatters the held gradients of `cell` and, when with_point, its point
    // gradient pg.  Lanes with the same cell are combined: every scattering
    // lane writes its record as a row of the LDS table, and for each group
    // (wave-uniform masks, lowest pending lane leading) the active lanes take
    // one column each, add it down the members' rows and send the sum with a
    // global atomic (a texture column once per run of members sharing its
    // tap).  A lone lane goes the same way: its record then leaves as one
    // atomic per column, spread over the active lanes.
    __device__ __forceinline__ void scatter(uint32_t cell, bool with_point, f3 pg)
    {
        const bool color = held_taps != HELD_NO_COLOR;
        const uint32_t lane = threadIdx.x & 63u;
        {
            float4 *row = reinterpret_cast<float4 *>(rows + lane * ROW_STRIDE);
            const float g0 = color ? held_gl[0] : 0.0f, g1 = color ? held_gl[1] : 0.0f,
                        g2 = color ? held_gl[2] : 0.0f;
            // diffuse taps 0-3, then specular taps 0-3, three channels each
            row[0] = make_float4(held_w[0] * g0, held_w[0] * g1, held_w[0] * g2, held_w[1] * g0);
            row[1] = make_float4(held_w[1] * g1, held_w[1] * g2, held_w[2] * g0, held_w[2] * g1);
            row[2] = make_float4(held_w[2] * g2, held_w[3] * g0, held_w[3] * g1, held_w[3] * g2);
            row[3] = make_float4(spec.w00 * g0, spec.w00 * g1, spec.w00 * g2, spec.w10 * g0);
            row[4] = make_float4(spec.w10 * g1, spec.w10 * g2, spec.w01 * g0, spec.w01 * g1);
            row[5] = make_float4(spec.w01 * g2, spec.w11 * g0, spec.w11 * g1, spec.w11 * g2);
            row[6] = make_float4(held_ds, held_perr, with_point ? pg.x : 0.0f, with_point ? pg.y : 0.0f);
            row[7] = make_float4(with_point ? pg.z : 0.0f, __uint_as_float(held_taps), __uint_as_float(spec_taps), 0.0f);
        }
        wave_lds_sync();
        const uint64_t act = __ballot(1);
        const uint32_t nact = (uint32_t)__popcll(act), arank = lane_rank(act);
        if (nact >= (uint32_t)REC_COLS)
            combine<true>(cell, act, nact, arank, lane);
        else
            combine<false>(cell, act, nact, arank, lane);
        wave_lds_sync(); // the rows are read before the next scatter rewrites them
    }

    // After the walk: a walk that ended without the transmittance stop
    // (no exit face, step cap) still owes its last cell's held gradients;
    // that cell's point gradient is not scattered (its exit term never came).
    __device__ __forceinline__ void finish()
    {
        if (prev_idx != NONE)
            scatter(prev_idx, false, mk(0.0f, 0.0f, 0.0f));
    }

    float pdens; // density of the current cell, loaded by begin_cell

    __device__ __forceinline__ void begin_cell(uint32_t cell) { pdens = density[cell]; }

    template <class St>
    __device__ __forceinline__ bool integrate(uint32_t cell, float t0, float t1, f3 p, f3 np, St &st)
    {
        float sig = pdens;
        f3 rgb = mk(0.0f, 0.0f, 0.0f);
        Bilinear db;
        bool has_color = false;
        if (sig > 1e-6f) {
            st.shade();
            rgb = tex.color(cell, o, d, t0, p, spec, db);
            has_color = true;
        }
        float dt = __builtin_fmaxf(t1 - t0, 0.0f);
        float alpha = 1.0f - vt_expf(-sig * dt);
        float w = T * alpha;
        float da_ds = dt * (1.0f - alpha);
        float da_ddt = 0.0f;
        if (dt > 0.0f)
            da_ddt = sig * (1.0f - alpha);

        acc = vfma(w, rgb, acc);

        f3 dL_drgb = mk(fwd_rgb_grad.x * w, fwd_rgb_grad.y * w, fwd_rgb_grad.z * w);
        f3 rest = divs(sub(fwd_rgb, acc), T * ((1.0f - alpha) + 1e-6f));
        float dL_dalpha = T * dot(sub(rgb, rest), fwd_rgb_grad);
        dL_dalpha = dL_dalpha + ((1.0f - fwd_alpha) * fwd_alpha_grad) / ((1.0f - alpha) + 1e-6f);

        float dL_ds = dL_dalpha * da_ds;
        float dL_ddt = dL_dalpha * da_ddt;
        float dL_dt0 = 0.0f;

        if (dist_grad != 0.0f) {
            float s0 = 1.0f - 1.0f / (1.0f + t0);
            float s1 = 1.0f - 1.0f / (1.0f + t1);
            float mid = 0.5f * (s0 + s1);
            float ds = s1 - s0;
            float Wm = W_run;
            float Sm = S_run;
            float Wp = (W_total - Wm) - w;
            float Sp = fma_(-w, mid, S_total - Sm);
            float dL_dw_raw = fma_(2.0f / 3.0f * w, ds, fma_(2.0f, fma_(-mid, Wp, Sp), 2.0f * fma_(mid, Wm, -Sm)));
            float dL_dw_outer = dL_dw_raw * dist_grad;
            float dL_dw_w = dL_dw_outer * w;
            float D_iplus = (D_total - D_running) - dL_dw_w;
            dL_ds = dL_ds + fma_(-dt, D_iplus, (dL_dw_outer * T) * da_ds);
            D_running = D_running + dL_dw_w;
            W_run = W_run + w;
            S_run = fma_(w, mid, S_run);
        }

        float nextT = T * (1.0f - alpha);
        while (qi < nq && nextT < qval) {
            float dg = depth_grad[qi] / sig;
            dL_dt0 = dL_dt0 + dg;
            dL_ds = dL_ds + (-dg * vt_logf(T / qval)) / sig;
            cur_depth_grad = cur_depth_grad - dg;
            qi++;
            if (qi < nq)
                qval = qthr[qi];
        }
        if (qi < nq) {
            dL_ds = fma_(-dt, cur_depth_grad, dL_ds);
            dL_ddt = fma_(-sig, cur_depth_grad, dL_ddt);
        }
        dL_dt0 = dL_dt0 + -dL_ddt;
        float dL_dt1 = dL_ddt;

        f3 dt0_dprev = mk(0.0f, 0.0f, 0.0f);
        if (prev_idx != NONE)
            dt0_dprev = cell_intersection_grad(prev_geom, p, o, d);
        f3 dt1_dcur = cell_intersection_grad(p, np, o, d);
        f3 dt0_dcur = cell_intersection_grad(p, prev_geom, o, d);
        f3 dt1_dnext = cell_intersection_grad(np, p, o, d);

        prev_grad = vfma(dL_dt0, dt0_dprev, prev_grad);
        f3 cg = mk(fma_(dL_dt1, dt1_dcur.x, dL_dt0 * dt0_dcur.x), fma_(dL_dt1, dt1_dcur.y, dL_dt0 * dt0_dcur.y),
                   fma_(dL_dt1, dt1_dcur.z, dL_dt0 * dt0_dcur.z));
        cur_grad = add(cur_grad, cg);
        next_grad = vfma(dL_dt1, dt1_dnext, next_grad);

        // the previous cell's held gradients and its now complete point gradient
        if (prev_idx != NONE)
            scatter(prev_idx, true, prev_grad);
        prev_geom = p;
        prev_idx = cell;
        prev_grad = cur_grad;
        cur_grad = next_grad;
        next_grad = mk(0.0f, 0.0f, 0.0f);

        T = nextT;

        float gl[3] = {0.0f, 0.0f, 0.0f};
        if (has_color) {
            gl[0] = (dL_drgb.x * rgb.x) * (1.0f - rgb.x);
            gl[1] = (dL_drgb.y * rgb.y) * (1.0f - rgb.y);
            gl[2] = (dL_drgb.z * rgb.z) * (1.0f - rgb.z);
        }
        hold(has_color, db, gl, dL_ds, w * ray_error);

        if (T < thr) {
            scatter(cell, true, prev_grad);
            prev_idx = NONE; // nothing held any more
            return false;
        }
        return true;
    }
};

template <typename A, int RD, int RS, bool STATS>
__global__ __launch_bounds__(TRAIN_BLOCK) __attribute__((amdgpu_waves_per_eu(TRAIN_BWD_WAVES)))
void bwd_kernel(BwdArgs a)
{
    __shared__ __align__(16) float rows_lds[TRAIN_WAVES][ROW_TABLE_FLOATS];
    float *rows = rows_lds[threadIdx.x / 64];
    if ((threadIdx.x & 63u) < (uint32_t)ROW_STRIDE)
        rows[64 * ROW_STRIDE + (threadIdx.x & 63u)] = 0.0f; // the zero row
    wave_lds_sync();
    uint32_t r = train_ray<false>(xcd_interleaved_block<TRAIN_XCD_CHUNK>() * blockDim.x + threadIdx.x, a.num_rays,
                                  a.ray_perm, a.num_images, a.img_h, a.img_w, a.tile_order);
    if (r == NONE)
        return;
    BwdIntegrator<A, RD, RS> it;
    it.rows = rows;
    load_ray(a.rays, r, it.o, it.d);
    it.density = a.density;
    it.tex.diffuse = (const A *)a.diffuse;
    it.tex.specular = (const A *)a.specular;
    float su, sv;
    oct_encode<RS>(mk(-it.d.x, -it.d.y, -it.d.z), su, sv);
    it.spec = bilinear_setup<RS>(su, sv);
    static_assert(RS * RS <= 256, "specular tap indices are packed in 8 bits");
    it.spec_taps = (uint32_t)it.spec.i00 | (uint32_t)it.spec.i10 << 8 | (uint32_t)it.spec.i01 << 16 |
                   (uint32_t)it.spec.i11 << 24;
    // a record of an unshaded cell writes held_w * 0 into the row
    it.held_w[0] = it.held_w[1] = it.held_w[2] = it.held_w[3] = 0.0f;
    it.thr = a.thr;
    const A *rg = (const A *)a.rgba_grad;
    const A *rv = (const A *)a.rgba;
    float g[4], v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        g[i] = Attr<A>::load(rg, 4 * (size_t)r + i);
        v[i] = Attr<A>::load(rv, 4 * (size_t)r + i);
    }
    g[3] = g[3] + a.contribution_alpha_grad;
    it.ray_error = a.ray_error ? Attr<A>::load((const A *)a.ray_error, r) : 0.0f;
    uint32_t K = a.quantiles ? a.K : 0;
    float cdg = 0.0f;
    for (uint32_t i = 0; i < K; ++i) {
        uint32_t q = a.depth_idx[(size_t)r * K + i];
        if (q != NONE)
            cdg = cdg + a.depth_grad[(size_t)r * K + i] / a.density[q];
    }
    it.acc = mk(0.0f, 0.0f, 0.0f);
    it.T = 1.0f;
    it.cur_depth_grad = cdg;
    it.qi = 0;
    it.nq = K;
    it.qthr = K ? a.quantiles + (size_t)r * K : nullptr;
    it.depth_grad = K ? a.depth_grad + (size_t)r * K : nullptr;
    it.qval = K ? it.qthr[0] : 0.0f;
    it.cell_grad = a.cell_grad;
    it.diffuse_grad = (A *)a.diffuse_grad;
    it.specular_grad = (A *)a.specular_grad;
    it.point_error = (A *)a.point_error;
    it.prev_geom = it.prev_grad = it.cur_grad = it.next_grad = mk(0.0f, 0.0f, 0.0f);
    it.prev_idx = NONE;
    it.fwd_rgb = mk(v[0], v[1], v[2]);
    it.fwd_alpha = v[3];
    it.fwd_rgb_grad = mk(g[0], g[1], g[2]);
    it.fwd_alpha_grad = g[3];
    it.W_run = it.S_run = it.D_running = 0.0f;
    it.W_total = a.W_total ? a.W_total[r] : 0.0f;
    it.S_total = a.S_total ? a.S_total[r] : 0.0f;
    float fd = a.distortion ? a.distortion[r] : 0.0f;
    it.dist_grad = a.distortion_grad ? a.distortion_grad[r] : 0.0f;
    it.D_total = (2.0f * fd) * it.dist_grad;
    StatsAcc<STATS> st;
    st.begin(a.stats, r);
    const uint32_t start = a.start_point[r];
    const uint32_t n = start < a.num_points ? walk<TRAIN_BWD_CHUNK>(it.o, it.d, a.points, a.adjacency, a.offsets,
                                                                    a.adj_diff, start, a.max_steps, it, st)
                                            : 0u;
    it.finish();
    st.store(a.stats, r, n);
}

int prefetch(const float *points, uint32_t num_points, const uint32_t *adjacency, uint32_t adjacency_size,
             const uint32_t *offsets, uint16_t *adj_diff, hipStream_t stream);

template <typename Args>
static void set_lane_order(Args &a, uint32_t num_rays, const uint32_t *ray_perm, uint32_t h, uint32_t w)
{
    a.ray_perm = ray_perm;
    a.num_images = 0;
    a.img_h = a.img_w = 0;
    uint64_t px = (uint64_t)h * w;
    if (!ray_perm && h && w && num_rays % px == 0) {
        a.num_images = (uint32_t)(num_rays / px);
        a.img_h = h;
        a.img_w = w;
    }
}

// Waves of a training kernel resident at once on the current device:
// waves_per_simd (its register budget, amdgpu_waves_per_eu) x 4 SIMDs per CU.
static uint32_t resident_waves(uint32_t waves_per_simd)
{
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return 0;
    return (uint32_t)cus * 4u * waves_per_simd;
}

template <typename A, int RD, int RS, bool ST> struct FwdK {
    static constexpr auto fn = fwd_kernel<A, RD, RS, ST>;
    static uint32_t resident() { return resident_waves(TRAIN_FWD_WAVES); }
};
template <typename A, int RD, int RS, bool ST> struct BwdK {
    static constexpr auto fn = bwd_kernel<A, RD, RS, ST>;
    static uint32_t resident() { return resident_waves(TRAIN_BWD_WAVES); }
};

template <template <typename, int, int, bool> class K, typename Args, typename A, int RD, int RS>
static int launch_train_rs(const Args &a, bool stats, hipStream_t s)
{
    uint64_t slots = a.num_rays;
    if (a.num_images || a.ray_perm) {
        const uint64_t tiles = train_tiles(a.num_rays, a.ray_perm != nullptr, a.num_images, a.img_h, a.img_w);
        slots = tiles * 64;
        // the waves that run split tiles' second halves (at most one per
        // resident wave: the split count stays below 1.25x that; see
        // vt_tile_order)
        if (a.tile_order)
            slots += std::min<uint64_t>(tiles, K<A, RD, RS, false>::resident()) * 64;
    }
    dim3 grid((uint32_t)((slots + TRAIN_BLOCK - 1) / TRAIN_BLOCK)), block(TRAIN_BLOCK);
    if (stats)
        hipLaunchKernelGGL((K<A, RD, RS, true>::fn), grid, block, 0, s, a);
    else
        hipLaunchKernelGGL((K<A, RD, RS, false>::fn), grid, block, 0, s, a);
    VT_LAUNCH_CHECK("training traversal kernel");
    return VT_OK;
}


template <template <typename, int, int, bool> class K, typename Args, typename A>
static int launch_train_a(const Args &a, uint32_t rd, uint32_t rs, bool stats, hipStream_t s)
{
    if (rd == 4 && rs == 4)
        return launch_train_rs<K, Args, A, 4, 4>(a, stats, s);
    if (rd == 8 && rs == 8)
        return launch_train_rs<K, Args, A, 8, 8>(a, stats, s);
    if (rd == 8 && rs == 4)
        return launch_train_rs<K, Args, A, 8, 4>(a, stats, s);
    if (rd == 4 && rs == 8)
        return launch_train_rs<K, Args, A, 4, 8>(a, stats, s);
    set_error("unsupported octahedral map resolution (diffuse %u, specular %u); compiled: 4, 8", rd, rs);
    return VT_ERR_UNSUPPORTED;
}

template <template <typename, int, int, bool> class K, typename Args>
static int launch_train(int attr_dtype, const Args &a, uint32_t rd, uint32_t rs, bool stats, hipStream_t s)
{
    if (a.num_rays == 0)
        return VT_OK;
    if (attr_dtype == VT_ATTR_F32)
        return launch_train_a<K, Args, float>(a, rd, rs, stats, s);
    if (attr_dtype == VT_ATTR_F16)
        return launch_train_a<K, Args, uint16_t>(a, rd, rs, stats, s);
    set_error("Unsupported color dtype. Only float32 and float16 are supported.");
    return VT_ERR_INVALID;
}

} // namespace vt

using namespace vt;

extern "C" int vt_trace_fwd(int attr_dtype, const float *points, const void *diffuse, const void *specular,
                            uint32_t diff_res, uint32_t spec_res, const float *density, const uint32_t *adjacency,
                            uint32_t adjacency_size, const uint32_t *offsets, uint32_t num_points, const float *rays,
                            uint32_t num_rays, uint32_t image_h, uint32_t image_w,
                            const uint32_t *start_point, const uint32_t *ray_perm, uint32_t num_quantiles,
                            const float *depth_quantiles, float weight_threshold, uint32_t max_intersections,
                            void *rgba, float *depth, uint32_t *depth_idx, void *contribution,
                            uint32_t *num_intersections, float *distortion, float *W_total, float *S_total,
                            float *t_far, uint16_t *adj_diff_workspace, const uint32_t *tile_order,
                            uint32_t *tile_cost, vt_ray_stats *stats, vt_stream_t stream)
{
    clear_error();
    VT_REQUIRE(points && diffuse && specular && density && adjacency && offsets && adj_diff_workspace,
               "null scene pointer");
    VT_REQUIRE(num_rays == 0 || (rays && start_point && rgba && distortion && W_total && S_total && t_far),
               "null ray or output pointer");
    VT_REQUIRE(!depth_quantiles || num_quantiles == 0 || (depth && depth_idx),
               "depth outputs required when depth_quantiles is given");
    VT_REQUIRE(num_rays == 0 || num_points > 0, "rays need at least one site");
    hipStream_t s = as_stream(stream);
    int rc = prefetch(points, num_points, adjacency, adjacency_size, offsets, adj_diff_workspace, s);
    if (rc)
        return rc;
    FwdArgs a{};
    a.points = points;
    a.diffuse = diffuse;
    a.specular = specular;
    a.density = density;
    a.adjacency = adjacency;
    a.offsets = offsets;
    a.adj_diff = reinterpret_cast<const uint2 *>(adj_diff_workspace);
    a.rays = rays;
    a.num_rays = num_rays;
    set_lane_order(a, num_rays, ray_perm, image_h, image_w);
    a.start_point = start_point;
    a.num_points = num_points;
    a.K = depth_quantiles ? num_quantiles : 0;
    a.quantiles = (depth_quantiles && num_quantiles) ? depth_quantiles : nullptr;
    a.thr = weight_threshold;
    a.max_steps = max_intersections;
    a.rgba = rgba;
    a.depth = depth;
    a.depth_idx = depth_idx;
    a.contribution = contribution;
    a.n_out = num_intersections;
    a.distortion = distortion;
    a.W_total = W_total;
    a.S_total = S_total;
    a.t_far = t_far;
    a.stats = reinterpret_cast<uint32_t *>(stats);
    // tiles exist for image lanes and for the waves of a ray_perm lane order
    const bool tiled = a.num_images || a.ray_perm;
    a.tile_order = tiled ? tile_order : nullptr;
    a.tile_cost = tiled ? tile_cost : nullptr;
    return launch_train<FwdK>(attr_dtype, a, diff_res, spec_res, stats != nullptr, s);
}

// The backward adds each cell's point and density gradients into one
// 16-byte slot (x, y, z, density) of the caller's workspace, so that a
// combined group's four sums there touch one cache line instead of one in
// points_grad and one in density_grad; the slots are then added into those
// outputs (caller zero-initialised, so the sums arrive unchanged).
__global__ void cell_grad_clear_kernel(float4 *g, uint32_t n)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        g[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

__global__ void cell_grad_out_kernel(const float4 *g, float *points_grad, float *density_grad, uint32_t n)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float4 v = g[i];
        points_grad[3 * (size_t)i + 0] += v.x;
        points_grad[3 * (size_t)i + 1] += v.y;
        points_grad[3 * (size_t)i + 2] += v.z;
        density_grad[i] += v.w;
    }
}

extern "C" int vt_trace_bwd(int attr_dtype, const float *points, const void *diffuse, const void *specular,
                            uint32_t diff_res, uint32_t spec_res, const float *density, const uint32_t *adjacency,
                            uint32_t adjacency_size, const uint32_t *offsets, uint32_t num_points, const float *rays,
                            uint32_t num_rays, uint32_t image_h, uint32_t image_w,
                            const uint32_t *start_point, const uint32_t *ray_perm, const void *rgba,
                            const void *rgba_grad,
                            uint32_t num_quantiles, const float *depth_quantiles, const uint32_t *depth_idx,
                            const float *depth_grad, const void *ray_error, float contribution_alpha_grad,
                            const float *distortion, const float *distortion_grad, const float *W_total,
                            const float *S_total, const float *t_far, float weight_threshold,
                            uint32_t max_intersections, float *points_grad, void *diffuse_grad, void *specular_grad,
                            float *density_grad, void *point_error, uint16_t *adj_diff_workspace,
                            int adj_diff_ready, float *cell_workspace, const uint32_t *tile_order,
                            vt_ray_stats *stats, vt_stream_t stream)
{
    clear_error();
    (void)t_far;
    VT_REQUIRE(points && diffuse && specular && density && adjacency && offsets && adj_diff_workspace,
               "null scene pointer");
    VT_REQUIRE(num_rays == 0 || (rays && start_point && rgba && rgba_grad), "null ray pointer");
    VT_REQUIRE(points_grad && diffuse_grad && specular_grad && density_grad, "null gradient output");
    VT_REQUIRE(cell_workspace && reinterpret_cast<uintptr_t>(cell_workspace) % 16 == 0,
               "cell_workspace must be a 16-byte aligned (num_points, 4) float array");
    VT_REQUIRE(!depth_quantiles || num_quantiles == 0 || (depth_idx && depth_grad),
               "depth_idx and depth_grad required when depth_quantiles is given");
    VT_REQUIRE(!ray_error || point_error, "point_error output required when ray_error is given");
    VT_REQUIRE(num_rays == 0 || num_points > 0, "rays need at least one site");
    hipStream_t s = as_stream(stream);
    int rc = VT_OK;
    if (!adj_diff_ready) // else the forward of the same scene filled it
        rc = prefetch(points, num_points, adjacency, adjacency_size, offsets, adj_diff_workspace, s);
    if (rc)
        return rc;
    BwdArgs a{};
    a.points = points;
    a.diffuse = diffuse;
    a.specular = specular;
    a.density = density;
    a.adjacency = adjacency;
    a.offsets = offsets;
    a.adj_diff = reinterpret_cast<const uint2 *>(adj_diff_workspace);
    a.rays = rays;
    a.num_rays = num_rays;
    set_lane_order(a, num_rays, ray_perm, image_h, image_w);
    a.start_point = start_point;
    a.num_points = num_points;
    a.rgba = rgba;
    a.rgba_grad = rgba_grad;
    a.K = depth_quantiles ? num_quantiles : 0;
    a.quantiles = (depth_quantiles && num_quantiles) ? depth_quantiles : nullptr;
    a.depth_idx = depth_idx;
    a.depth_grad = depth_grad;
    a.ray_error = ray_error;
    a.contribution_alpha_grad = contribution_alpha_grad;
    a.distortion = distortion;
    a.distortion_grad = distortion_grad;
    a.W_total = W_total;
    a.S_total = S_total;
    a.thr = weight_threshold;
    a.max_steps = max_intersections;
    a.cell_grad = cell_workspace;
    a.diffuse_grad = diffuse_grad;
    a.specular_grad = specular_grad;
    a.point_error = point_error;
    a.stats = reinterpret_cast<uint32_t *>(stats);
    a.tile_order = (a.num_images || a.ray_perm) ? tile_order : nullptr;
    if (num_rays == 0)
        return VT_OK;
    const uint32_t cblocks = (num_points + 255) / 256;
    cell_grad_clear_kernel<<<cblocks, 256, 0, s>>>(reinterpret_cast<float4 *>(cell_workspace), num_points);
    VT_LAUNCH_CHECK("cell_grad_clear_kernel");
    rc = launch_train<BwdK>(attr_dtype, a, diff_res, spec_res, stats != nullptr, s);
    if (rc)
        return rc;
    cell_grad_out_kernel<<<cblocks, 256, 0, s>>>(reinterpret_cast<const float4 *>(cell_workspace), points_grad,
                                                  density_grad, num_points);
    VT_LAUNCH_CHECK("cell_grad_out_kernel");
    return VT_OK;
}

// ---- self-test of the half-precision atomic --------------------------------

namespace vt {

__global__ void f16_atomic_probe_kernel(uint16_t *halves, uint32_t num_halves, const uint32_t *__restrict__ index,
                                        const float *__restrict__ values, uint32_t n)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n && index[i] < num_halves)
        Attr<uint16_t>::add(halves, index[i], values[i]);
}

} // namespace vt

extern "C" uint32_t vt_train_fwd_resident_waves(void)
{
    return vt::resident_waves(vt::TRAIN_FWD_WAVES);
}

extern "C" uint32_t vt_train_bwd_resident_waves(void)
{
    return vt::resident_waves(vt::TRAIN_BWD_WAVES);
}

extern "C" int vt_debug_f16_atomic_add(uint16_t *halves, uint32_t num_halves, const uint32_t *index,
                                       const float *values, uint32_t n, vt_stream_t stream)
{
    clear_error();
    VT_REQUIRE(num_halves % 2 == 0, "num_halves must be even (whole 32-bit words), got %u", num_halves);
    if (n == 0)
        return VT_OK;
    VT_REQUIRE(halves && index && values, "null pointer argument");
    VT_REQUIRE(((uintptr_t)halves & 3u) == 0, "halves must be 4-byte aligned");
    f16_atomic_probe_kernel<<<(n + 255) / 256, 256, 0, as_stream(stream)>>>(halves, num_halves, index, values, n);
    VT_LAUNCH_CHECK("f16_atomic_probe_kernel");
    return VT_OK;
}
