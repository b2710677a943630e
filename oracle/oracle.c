/*
 * oracle.c -- CPU restatement of the VoroTracing traversal hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for the HIP library,
 * never part of it.  Build: oracle/Makefile (gcc -O3 -fopenmp
 * -ffp-contract=off, no fast-math).
 *
 * Reference files restated here (paths under /root/reference):
 *   vorotracing/cuda/csrc/tracing/tracing_octmap.cu
 *       :39-123   trace_octmap (the cell walk)                -> walk()
 *       :125-149  prefetch_adjacent_diff_octmap_kernel        -> or_prefetch_adj
 *       :175-229  trace_vorotracing_fwd_kernel body            -> or_trace_fwd
 *       :264-339  trace_vorotracing_bwd_kernel body            -> or_trace_bwd
 *       :567-609  trace_vorotracing_infer_kernel body          -> or_trace_infer_f16
 *       :741-778  trace_vorotracing_infer_q8_kernel body       -> or_trace_infer_q8
 *   vorotracing/cuda/csrc/tracing/ray_integrator_octmap.cuh
 *       :17-35    oct_encode, :37-55 oct_wrap_index
 *       :102-152, :251-281   RayIntegratorOctMap (training fwd)
 *       :315-344, :437-460   RayIntegratorOctMapInfer (fp16)
 *       :487-515, :536, :609-632 RayIntegratorOctMapInferQ8
 *       :683-860, :979-1026  RayIntegratorOctMapBackward
 *   vorotracing/cuda/csrc/tracing/ray_integrator.cuh:39-53  cell_intersection_grad
 *   vorotracing/cuda/csrc/utils/typing.cuh:18-24  f16 casts (RNE)
 *   vorotracing/cuda/csrc/utils/geometry.h:123-129 atomic_add_vec (atomics kept)
 *   vorotracing/utils/__init__.py:85-130, vorotracing/datasets/datasets.py
 *       :126-136, :286-304  camera rays                         -> or_camera_rays
 *
 * Parity pins (tests/test_oracle_*.py): f16 casts vs numpy.float16 (all
 * halves, random floats); or_expf/or_logf vs float64 libm (<= 2 ulp); walk vs
 * closed-form cubic lattices, two-site scenes and brute-force nearest-site on
 * exact-in-fp16 scenes; compositing vs closed forms; distortion vs the O(n^2)
 * definition; backward vs float64 central differences; Morton / tile
 * permutation invariance.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define OR_NONE 0xffffffffu

/* planted mistake for the pin tests (oracle.h); 0 in every other use */
static int g_plant = OR_PLANT_NONE;
void or_set_plant(int code) { g_plant = code; }
int or_get_plant(void) { return g_plant; }

/* absolute-sum mode (oracle.h): every atomic add adds |v| (1), or 1 (2); 0 in every other use */
static int g_abs_sums = 0;
void or_set_abs_sums(int on) { g_abs_sums = on; }
static inline float sum_mode_value(float v) { return g_abs_sums == 2 ? 1.0f : fabsf(v); }

/* ------------------------------------------------------------------------- */
/* scalar math                                                                 */
/* ------------------------------------------------------------------------- */

static inline float bits_f(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static inline uint32_t f_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* f32 -> f16, round to nearest even (the __float2half of typing.cuh:24). */
uint16_t or_f32_to_f16(float f)
{
    uint32_t x = f_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) /* NaN: keep quiet NaN with top payload bits */
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) /* >= 65520 rounds to infinity (incl. inf) */
        return (uint16_t)(sign | 0x7c00u);
    if (ax >= 0x38800000u) { /* result is a normal half */
        uint32_t e = (ax >> 23) - 127u + 15u;
        uint32_t m = ax & 0x7fffffu;
        uint32_t h = (e << 10) | (m >> 13);
        uint32_t rem = m & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u)))
            h += 1u;
        return (uint16_t)(sign | h);
    }
    /* subnormal half or zero: units of 2^-24, scaling by 2^24 is exact */
    float scaled = bits_f(ax) * 16777216.0f;
    return (uint16_t)(sign | (uint16_t)rintf(scaled));
}

float or_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0x1fu)
        return bits_f(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        float v = (float)m * (1.0f / 16777216.0f);
        return sign ? -v : v;
    }
    return bits_f(sign | ((e + 112u) << 23) | (m << 13));
}

/*
 * exp(x): Cody & Waite (1980) two-constant range reduction x = k ln2 + r,
 * |r| <= ln2/2, then the degree-7 Taylor polynomial of e^r (remainder
 * < 6e-9 relative), then scaling by 2^k with one final rounding.  The split
 * of ln2 is ln2 rounded to 16 fractional bits (so k*LN2_HI is exact) plus the
 * float nearest to the remainder.
 */
#define OR_LOG2E 1.44269502162933349609375f
#define OR_LN2_HI 0.693145751953125f
#define OR_LN2_LO 1.42860676533018704e-06f

float or_expf(float x)
{
    if (x != x)
        return x;
    if (x > 88.72283935546875f)
        return INFINITY;
    if (x < -103.972084045410156f)
        return 0.0f;
    float kf = rintf(x * OR_LOG2E);
    float r = fmaf(kf, -OR_LN2_HI, x);
    r = fmaf(kf, -OR_LN2_LO, r);
    float q = 1.0f / 5040.0f;
    q = fmaf(q, r, 1.0f / 720.0f);
    q = fmaf(q, r, 1.0f / 120.0f);
    q = fmaf(q, r, 1.0f / 24.0f);
    q = fmaf(q, r, 1.0f / 6.0f);
    q = fmaf(q, r, 0.5f);
    float e = fmaf(q, r * r, r) + 1.0f;
    int k = (int)kf;
    if (k > 127)
        return (e * bits_f(0x7f000000u)) * bits_f((uint32_t)(k - 127 + 127) << 23);
    if (k < -126)
        return (e * bits_f((uint32_t)(k + 64 + 127) << 23)) * bits_f((uint32_t)(-64 + 127) << 23);
    return e * bits_f((uint32_t)(k + 127) << 23);
}

/*
 * log(x): x = 2^e m with m in [sqrt(1/2), sqrt(2)), s = (m-1)/(m+1),
 * log m = 2 atanh s = 2s + 2s^3/3 + ... + 2s^11/11 (|s| <= 0.1716), then
 * e*ln2 with the Cody-Waite split above.
 */
float or_logf(float x)
{
    if (x != x || x < 0.0f)
        return NAN;
    if (x == 0.0f)
        return -INFINITY;
    if (x == INFINITY)
        return x;
    int eadj = 0;
    if (x < 1.17549435e-38f) {
        x *= 8388608.0f;
        eadj = -23;
    }
    uint32_t b = f_bits(x);
    int e = (int)((b >> 23) & 0xffu) - 127 + eadj;
    float m = bits_f((b & 0x7fffffu) | 0x3f800000u);
    if (m > 1.41421356f) {
        m *= 0.5f;
        e += 1;
    }
    float f = m - 1.0f;
    float s = f / (f + 2.0f);
    float z = s * s;
    float p = 2.0f / 11.0f;
    p = fmaf(p, z, 2.0f / 9.0f);
    p = fmaf(p, z, 2.0f / 7.0f);
    p = fmaf(p, z, 2.0f / 5.0f);
    p = fmaf(p, z, 2.0f / 3.0f);
    float lm = fmaf(s * z, p, 2.0f * s);
    float ef = (float)e;
    return fmaf(ef, OR_LN2_HI, fmaf(ef, OR_LN2_LO, lm));
}

void or_expf_many(const float *x, float *y, size_t n)
{
    for (size_t i = 0; i < n; ++i)
        y[i] = or_expf(x[i]);
}
void or_logf_many(const float *x, float *y, size_t n)
{
    for (size_t i = 0; i < n; ++i)
        y[i] = or_logf(x[i]);
}
void or_f32_to_f16_many(const float *x, uint16_t *y, size_t n)
{
    for (size_t i = 0; i < n; ++i)
        y[i] = or_f32_to_f16(x[i]);
}

/* ------------------------------------------------------------------------- */
/* vectors                                                                     */
/* ------------------------------------------------------------------------- */

typedef struct { float x, y, z; } v3;

static inline v3 mk(float x, float y, float z) { v3 r = {x, y, z}; return r; }
static inline v3 vsub(v3 a, v3 b) { return mk(a.x - b.x, a.y - b.y, a.z - b.z); }
static inline v3 vadd(v3 a, v3 b) { return mk(a.x + b.x, a.y + b.y, a.z + b.z); }
static inline v3 vscale(float s, v3 a) { return mk(s * a.x, s * a.y, s * a.z); }
static inline v3 vdivs(v3 a, float s) { return mk(a.x / s, a.y / s, a.z / s); }
static inline float vdot(v3 a, v3 b) { return fmaf(a.z, b.z, fmaf(a.y, b.y, a.x * b.x)); }
/* acc + s*a, contracted (Eigen "acc += s * a") */
static inline v3 vfma(float s, v3 a, v3 acc)
{
    return mk(fmaf(s, a.x, acc.x), fmaf(s, a.y, acc.y), fmaf(s, a.z, acc.z));
}
static inline v3 ld3(const float *p, uint32_t i) { return mk(p[3 * (size_t)i], p[3 * (size_t)i + 1], p[3 * (size_t)i + 2]); }

/* ------------------------------------------------------------------------- */
/* octahedral map (ray_integrator_octmap.cuh:17-55)                           */
/* ------------------------------------------------------------------------- */

int or_oct_wrap_index(int u, int v, int R)
{
    if (u >= 0 && u < R && v >= 0 && v < R)
        return v * R + u;
    int wu = ((u % R) + R) % R;
    int wv = ((v % R) + R) % R;
    int fu = abs(u / R) + (u < 0 ? 1 : 0);
    int fv = abs(v / R) + (v < 0 ? 1 : 0);
    if (((fu ^ fv) & 1) != 0) {
        wu = R - 1 - wu;
        wv = R - 1 - wv;
    }
    return wv * R + wu;
}

static inline void oct_encode(v3 d, int R, float *tu, float *tv)
{
    float l1 = (fabsf(d.x) + fabsf(d.y)) + fabsf(d.z);
    float inv = 1.0f / fmaxf(l1, 1e-10f);
    float u = d.x * inv;
    float v = d.y * inv;
    if (d.z < 0.0f) {
        float ou = (1.0f - fabsf(v)) * copysignf(1.0f, u);
        float ov = (1.0f - fabsf(u)) * copysignf(1.0f, v);
        u = ou;
        v = ov;
    }
    *tu = fmaf(fmaf(u, 0.5f, 0.5f), (float)R, -0.5f);
    *tv = fmaf(fmaf(v, 0.5f, 0.5f), (float)R, -0.5f);
}

void or_oct_encode(const float dir[3], int R, float uv[2])
{
    oct_encode(mk(dir[0], dir[1], dir[2]), R, &uv[0], &uv[1]);
}

/* bilinear taps + weights (e.g. ray_integrator_octmap.cuh:200-221) */
typedef struct {
    int i00, i10, i01, i11;
    float w00, w10, w01, w11;
} bil_t;

static inline bil_t bil_setup(float u, float v, int R)
{
    bil_t b;
    int u0 = (int)floorf(u);
    int v0 = (int)floorf(v);
    float fu = u - (float)u0;
    float fv = v - (float)v0;
    b.i00 = or_oct_wrap_index(u0, v0, R);
    b.i10 = or_oct_wrap_index(u0 + 1, v0, R);
    b.i01 = or_oct_wrap_index(u0, v0 + 1, R);
    b.i11 = or_oct_wrap_index(u0 + 1, v0 + 1, R);
    b.w00 = (1.0f - fu) * (1.0f - fv);
    b.w10 = fu * (1.0f - fv);
    b.w01 = (1.0f - fu) * fv;
    b.w11 = fu * fv;
    return b;
}

/* w00*a + w10*b + w01*c + w11*d, left to right, contracted */
static inline float bil_mix(const bil_t *b, float a, float bb, float c, float d)
{
    return fmaf(b->w11, d, fmaf(b->w01, c, fmaf(b->w10, bb, b->w00 * a)));
}

static inline float sigmoid(float x) { return 1.0f / (1.0f + or_expf(-x)); }

/* the diffuse probe direction (ray_integrator_octmap.cuh:258-264, :440-446) */
static inline v3 probe_dir(v3 o, v3 d, float t0, v3 site)
{
    v3 hit = mk(fmaf(t0, d.x, o.x), fmaf(t0, d.y, o.y), fmaf(t0, d.z, o.z));
    v3 dv = vsub(hit, site);
    float len = sqrtf(vdot(dv, dv));
    if (len > 1e-8f)
        return vdivs(dv, len);
    return d;
}

/* texel fetchers: channel c of texel i of cell `cell` */
typedef struct {
    int kind; /* 0 = f32 (N,3RR), 1 = f16 (N,3RR), 2 = f16 Half4Texel (N,4RR), 3 = u8 (N,3RR) */
    const void *base;
    int R;
    float scale[3], offset[3]; /* q8 only */
} texmap_t;

static inline float tex_fetch(const texmap_t *m, uint32_t cell, int i, int c)
{
    size_t RR = (size_t)m->R * (size_t)m->R;
    switch (m->kind) {
    case 0:
        return ((const float *)m->base)[cell * 3 * RR + (size_t)i * 3 + c];
    case 1:
        return or_f16_to_f32(((const uint16_t *)m->base)[cell * 3 * RR + (size_t)i * 3 + c]);
    case 2:
        return or_f16_to_f32(((const uint16_t *)m->base)[cell * 4 * RR + (size_t)i * 4 + c]);
    default: {
        uint8_t q = ((const uint8_t *)m->base)[cell * 3 * RR + (size_t)i * 3 + c];
        return fmaf(m->scale[c], (float)q, m->offset[c]); /* :536 scale*q + offset */
    }
    }
}

static inline v3 bil_sample(const texmap_t *m, uint32_t cell, const bil_t *b)
{
    float r[3];
    for (int c = 0; c < 3; ++c)
        r[c] = bil_mix(b, tex_fetch(m, cell, b->i00, c), tex_fetch(m, cell, b->i10, c),
                       tex_fetch(m, cell, b->i01, c), tex_fetch(m, cell, b->i11, c));
    return mk(r[0], r[1], r[2]);
}

/* colour of a cell: sigmoid(diffuse(probe) + specular(-d)) */
static inline v3 cell_color(const texmap_t *dm, const texmap_t *sm, const bil_t *spec, uint32_t cell, v3 o,
                            v3 d, float t0, v3 site, bil_t *diff_out)
{
    v3 pd = probe_dir(o, d, t0, site);
    float u, v;
    oct_encode(pd, dm->R, &u, &v);
    bil_t db = bil_setup(u, v, dm->R);
    if (diff_out)
        *diff_out = db;
    v3 a = bil_sample(dm, cell, &db);
    v3 b = bil_sample(sm, cell, spec);
    v3 logit = vadd(a, b);
    return mk(sigmoid(logit.x), sigmoid(logit.y), sigmoid(logit.z));
}

/* ------------------------------------------------------------------------- */
/* the walk (tracing_octmap.cu:39-123)                                        */
/* ------------------------------------------------------------------------- */

typedef struct {
    or_ray_stats st;
    uint32_t *log;
    uint32_t log_cap;
    uint32_t next; /* the cell behind the exit face of the step being integrated */
} walk_dbg_t;

typedef int (*integrate_fn)(void *state, uint32_t cell, float t0, float t1, v3 p, v3 np);

static inline void dbg_visit(walk_dbg_t *g, uint32_t cell)
{
    if (g->log && g->st.visits < g->log_cap)
        g->log[g->st.visits] = cell;
    if (g->st.visits < OR_STATS_LOG)
        g->st.first_cells[g->st.visits] = cell;
    g->st.visits += 1;
    g->st.visit_hash = (g->st.visit_hash ^ (uint64_t)cell) * 1099511628211ull;
}

/* Exit face of a cell with face records fl[0, nf) (tracing_octmap.cu:73-100):
 * the lowest j with dp > 0 minimising t = ((p + off/2 - o) . off) / dp, with
 * the reference's strict t < t_1 from t_1 = +inf.  *t1 = that t. */
static inline uint32_t exit_face(const uint16_t *fl, uint32_t nf, v3 p, v3 o, v3 d, float *t1_out)
{
    float t1 = INFINITY;
    uint32_t best = OR_NONE;
    for (uint32_t j = 0; j < nf; ++j) {
        const uint16_t *h = fl + 4 * (size_t)j;
        v3 off = mk(or_f16_to_f32(h[0]), or_f16_to_f32(h[1]), or_f16_to_f32(h[2]));
        v3 fo = mk(p.x + off.x * 0.5f, p.y + off.y * 0.5f, p.z + off.z * 0.5f);
        float dp = vdot(off, d);
        float t = vdot(vsub(fo, o), off) / dp;
        if (dp > 0.0f && t < t1) {
            t1 = t;
            best = j;
        }
    }
    *t1_out = t1;
    return best;
}

/* rows of 26 floats: site (3), origin (3), unit direction (3), face count
 * (u32 bits; counts above 8 read as 8), 8 face records of 4 halves (16
 * words); out: face index and t1 bits (0 when no face) per row. */
void or_exit_face_many(const float *rows, size_t n, uint32_t *out)
{
    for (size_t i = 0; i < n; ++i) {
        const float *r = rows + 26 * i;
        uint32_t nf = f_bits(r[9]);
        if (nf > 8)
            nf = 8;
        float t1 = 0.0f;
        uint32_t best = exit_face((const uint16_t *)(r + 10), nf, mk(r[0], r[1], r[2]), mk(r[3], r[4], r[5]),
                                  mk(r[6], r[7], r[8]), &t1);
        out[2 * i] = best;
        out[2 * i + 1] = best == OR_NONE ? 0u : f_bits(t1);
    }
}

static inline uint32_t walk(v3 o, v3 d, const float *points, const uint32_t *adjacency, const uint32_t *offsets,
                            const uint16_t *adj_diff, uint32_t start, uint32_t max_steps, integrate_fn integrate,
                            void *state, walk_dbg_t *g)
{
    float t0 = 0.0f;
    uint32_t n = 0;
    uint32_t cur = start;
    v3 p = ld3(points, cur);
    for (;;) {
        n++;
        if (n > max_steps)
            break;
        uint32_t b = offsets[cur];
        uint32_t e = offsets[cur + 1];
        uint32_t nf = e - b;
        dbg_visit(g, cur);
        g->st.faces += nf;
        float t1;
        uint32_t best = exit_face(adj_diff + 4 * (size_t)b, nf, p, o, d, &t1);
        if (best == OR_NONE)
            break;
        g->st.exits += 1;
        uint32_t nxt = adjacency[b + best];
        v3 np = ld3(points, nxt);
        if (t1 > t0) {
            g->st.integrated += 1;
            g->next = nxt;
            if (!integrate(state, cur, t0, t1, p, np))
                break;
        }
        t0 = fmaxf(t0, t1);
        cur = nxt;
        p = np;
    }
    g->st.n = n;
    return n;
}

static inline void read_ray(const float *rays, uint32_t r, v3 *o, v3 *d)
{
    const float *q = rays + 6 * (size_t)r;
    *o = mk(q[0], q[1], q[2]);
    v3 dd = mk(q[3], q[4], q[5]);
    float nrm = sqrtf(vdot(dd, dd)); /* ray.direction /= ray.direction.norm() */
    *d = vdivs(dd, nrm);
}

static inline void spec_setup(v3 d, int R, bil_t *b)
{
    float u, v;
    if (g_plant == OR_PLANT_SPEC_PLUS_D)
        oct_encode(d, R, &u, &v);
    else
        oct_encode(mk(-d.x, -d.y, -d.z), R, &u, &v);
    *b = bil_setup(u, v, R);
}

static void init_dbg(walk_dbg_t *g, uint32_t *log, uint32_t cap)
{
    memset(&g->st, 0, sizeof(g->st));
    g->st.visit_hash = 1469598103934665603ull;
    for (int i = 0; i < OR_STATS_LOG; ++i)
        g->st.first_cells[i] = OR_NONE;
    g->log = log;
    g->log_cap = cap;
    if (log)
        for (uint32_t i = 0; i < cap; ++i)
            log[i] = OR_NONE;
}

static int set_threads(int num_threads)
{
#ifdef _OPENMP
    if (num_threads > 0)
        return num_threads;
    return omp_get_max_threads();
#else
    (void)num_threads;
    return 1;
#endif
}

/* ------------------------------------------------------------------------- */
/* prefetch (tracing_octmap.cu:125-149)                                       */
/* ------------------------------------------------------------------------- */

void or_prefetch_adj(const float *points, uint32_t num_points, const uint32_t *adjacency, const uint32_t *offsets,
                     uint16_t *adj_diff, int num_threads)
{
    int nt = set_threads(num_threads);
#pragma omp parallel for schedule(dynamic, 1024) num_threads(nt)
    for (int64_t i = 0; i < (int64_t)num_points; ++i) {
        v3 p = ld3(points, (uint32_t)i);
        for (uint32_t e = offsets[i]; e < offsets[i + 1]; ++e) {
            v3 q = ld3(points, adjacency[e]);
            v3 df = vsub(q, p);
            uint16_t *h = adj_diff + 4 * (size_t)e;
            h[0] = or_f32_to_f16(df.x);
            h[1] = or_f32_to_f16(df.y);
            h[2] = or_f32_to_f16(df.z);
            h[3] = 0;
        }
    }
}

/* ------------------------------------------------------------------------- */
/* inference integrators (ray_integrator_octmap.cuh:315-344, :487-515)        */
/* ------------------------------------------------------------------------- */

typedef struct {
    v3 o, d;
    const float *density;
    texmap_t dm, sm;
    bil_t spec;
    float thr, skip;
    v3 acc;
    float T;
    walk_dbg_t *g;
} infer_state;

static int infer_integrate(void *sp, uint32_t cell, float t0, float t1, v3 p, v3 np)
{
    (void)np;
    infer_state *s = (infer_state *)sp;
    float sig = s->density[cell];
    if (sig <= 1e-6f && g_plant != OR_PLANT_INFER_NO_DENSITY_GATE)
        return s->T > s->thr;
    float dt = fmaxf(t1 - t0, 0.0f);
    float alpha = 1.0f - or_expf(-sig * dt);
    float w = s->T * alpha;
    if ((g_plant == OR_PLANT_SKIP_ON_ALPHA ? alpha : w) >= s->skip) {
        s->g->st.shaded += 1;
        v3 rgb = cell_color(&s->dm, &s->sm, &s->spec, cell, s->o, s->d, t0, p, NULL);
        s->acc = vfma(w, rgb, s->acc);
    }
    s->T = s->T * (1.0f - alpha);
    return s->T > s->thr;
}

static void trace_infer_common(const texmap_t *dm, const texmap_t *sm, const float *points, const float *density,
                               const uint32_t *adjacency, const uint32_t *offsets, const uint16_t *adj_diff,
                               const float *rays, uint32_t num_rays, const uint32_t *start_point,
                               const uint32_t *ray_perm, float thr, uint32_t max_int, float skip, uint16_t *rgba,
                               or_ray_stats *stats, uint32_t *visits_out, uint32_t max_log, int num_threads)
{
    int nt = set_threads(num_threads);
#pragma omp parallel for schedule(dynamic, 64) num_threads(nt)
    for (int64_t t = 0; t < (int64_t)num_rays; ++t) {
        uint32_t r = ray_perm ? ray_perm[t] : (uint32_t)t;
        infer_state s;
        walk_dbg_t g;
        init_dbg(&g, visits_out ? visits_out + (size_t)r * max_log : NULL, max_log);
        read_ray(rays, r, &s.o, &s.d);
        s.density = density;
        s.dm = *dm;
        s.sm = *sm;
        spec_setup(s.d, sm->R, &s.spec);
        s.thr = thr;
        s.skip = skip;
        s.acc = mk(0.0f, 0.0f, 0.0f);
        s.T = 1.0f;
        s.g = &g;
        walk(s.o, s.d, points, adjacency, offsets, adj_diff, start_point[r], max_int, infer_integrate, &s, &g);
        uint16_t *out = rgba + 4 * (size_t)r;
        out[0] = or_f32_to_f16(s.acc.x);
        out[1] = or_f32_to_f16(s.acc.y);
        out[2] = or_f32_to_f16(s.acc.z);
        out[3] = or_f32_to_f16(1.0f - s.T);
        if (stats)
            stats[r] = g.st;
    }
}

void or_trace_infer_f16(const float *points, const uint16_t *diffuse, const uint16_t *specular, int diff_res,
                        int spec_res, const float *density, const uint32_t *adjacency, const uint32_t *offsets,
                        const uint16_t *adj_diff, const float *rays, uint32_t num_rays, const uint32_t *start_point,
                        const uint32_t *ray_perm, float weight_threshold, uint32_t max_intersections,
                        float cell_skip_threshold, uint16_t *rgba, or_ray_stats *stats, uint32_t *visits_out,
                        uint32_t max_log, int num_threads)
{
    texmap_t dm = {2, diffuse, diff_res, {0, 0, 0}, {0, 0, 0}};
    texmap_t sm = {2, specular, spec_res, {0, 0, 0}, {0, 0, 0}};
    trace_infer_common(&dm, &sm, points, density, adjacency, offsets, adj_diff, rays, num_rays, start_point, ray_perm,
                       weight_threshold, max_intersections, cell_skip_threshold, rgba, stats, visits_out, max_log,
                       num_threads);
}

void or_trace_infer_q8(const float *points, const uint8_t *diffuse, const uint8_t *specular, int diff_res,
                       int spec_res, const float diff_scale[3], const float diff_offset[3], const float spec_scale[3],
                       const float spec_offset[3], const float *density, const uint32_t *adjacency,
                       const uint32_t *offsets, const uint16_t *adj_diff, const float *rays, uint32_t num_rays,
                       const uint32_t *start_point, float weight_threshold, uint32_t max_intersections,
                       float cell_skip_threshold, uint16_t *rgba, or_ray_stats *stats, int num_threads)
{
    texmap_t dm = {3, diffuse, diff_res, {0, 0, 0}, {0, 0, 0}};
    texmap_t sm = {3, specular, spec_res, {0, 0, 0}, {0, 0, 0}};
    for (int c = 0; c < 3; ++c) {
        dm.scale[c] = diff_scale[c];
        dm.offset[c] = diff_offset[c];
        sm.scale[c] = spec_scale[c];
        sm.offset[c] = spec_offset[c];
    }
    trace_infer_common(&dm, &sm, points, density, adjacency, offsets, adj_diff, rays, num_rays, start_point, NULL,
                       weight_threshold, max_intersections, cell_skip_threshold, rgba, stats, NULL, 0, num_threads);
}

/* ------------------------------------------------------------------------- */
/* atomics standing in for the reference's atomicAdd                           */
/* ------------------------------------------------------------------------- */

static inline void atomic_add_f32(float *dst, float v)
{
    if (g_abs_sums)
        v = sum_mode_value(v);
#pragma omp atomic
    *dst += v;
}

/* atomicAdd on a __half: CAS on the containing aligned 32-bit word */
static inline void atomic_add_f16(uint16_t *dst, float v)
{
    if (g_abs_sums)
        v = sum_mode_value(v);
    uintptr_t a = (uintptr_t)dst;
    uint32_t *word = (uint32_t *)(a & ~(uintptr_t)3);
    int hi = (a & 2) != 0;
    uint32_t old = __atomic_load_n(word, __ATOMIC_RELAXED);
    for (;;) {
        uint16_t h = hi ? (uint16_t)(old >> 16) : (uint16_t)(old & 0xffffu);
        uint16_t nh = or_f32_to_f16(or_f16_to_f32(h) + or_f16_to_f32(or_f32_to_f16(v)));
        uint32_t nw = hi ? ((old & 0x0000ffffu) | ((uint32_t)nh << 16)) : ((old & 0xffff0000u) | nh);
        if (__atomic_compare_exchange_n(word, &old, nw, 0, __ATOMIC_RELAXED, __ATOMIC_RELAXED))
            return;
    }
}

static inline void attr_atomic_add(int f16, void *base, size_t idx, float v)
{
    if (f16)
        atomic_add_f16((uint16_t *)base + idx, v);
    else
        atomic_add_f32((float *)base + idx, v);
}

static inline float attr_load(int f16, const void *base, size_t idx)
{
    return f16 ? or_f16_to_f32(((const uint16_t *)base)[idx]) : ((const float *)base)[idx];
}

static inline void attr_store(int f16, void *base, size_t idx, float v)
{
    if (f16)
        ((uint16_t *)base)[idx] = or_f32_to_f16(v);
    else
        ((float *)base)[idx] = v;
}

/* ------------------------------------------------------------------------- */
/* training forward (ray_integrator_octmap.cuh:102-152, :251-281)             */
/* ------------------------------------------------------------------------- */

typedef struct {
    v3 o, d;
    const float *density;
    texmap_t dm, sm;
    bil_t spec;
    float thr;
    int f16;
    void *contribution;
    const float *qthr;
    uint32_t nq, qi;
    float qval;
    float *qdepth;
    uint32_t *qidx;
    v3 acc;
    float T, W, S, D, self, tfar;
    walk_dbg_t *g;
} fwd_state;

static int fwd_integrate(void *sp, uint32_t cell, float t0, float t1, v3 p, v3 np)
{
    (void)np;
    fwd_state *s = (fwd_state *)sp;
    float sig = s->density[cell];
    v3 rgb = mk(0.0f, 0.0f, 0.0f);
    if (sig > 1e-6f) {
        s->g->st.shaded += 1;
        rgb = cell_color(&s->dm, &s->sm, &s->spec, cell, s->o, s->d, t0, p, NULL);
    }
    float dt = fmaxf(t1 - t0, 0.0f);
    float alpha = 1.0f - or_expf(-sig * dt);
    float w = s->T * alpha;

    float s0 = 1.0f - 1.0f / (1.0f + t0);
    float s1 = 1.0f - 1.0f / (1.0f + t1);
    float mid = 0.5f * (s0 + s1);
    float ds = s1 - s0;
    s->D = fmaf(w, fmaf(mid, s->W, -s->S), s->D);
    s->self = fmaf(w * w, ds, s->self);
    s->W = s->W + w;
    s->S = fmaf(w, mid, s->S);
    if (t1 > s->tfar)
        s->tfar = t1;

    if (s->contribution)
        attr_atomic_add(s->f16, s->contribution, cell, w);
    s->acc = vfma(w, rgb, s->acc);

    float nextT = s->T * (1.0f - alpha);
    while (s->qi < s->nq && nextT < s->qval) {
        s->qdepth[s->qi] = t0 + or_logf(s->T / s->qval) / sig;
        s->qidx[s->qi] = cell;
        s->qi++;
        if (s->qi < s->nq)
            s->qval = s->qthr[s->qi];
    }
    s->T = nextT;
    return s->T > s->thr;
}

void or_trace_fwd(int attr_f16, const float *points, const void *diffuse, const void *specular, int diff_res,
                  int spec_res, const float *density, const uint32_t *adjacency, const uint32_t *offsets,
                  const uint16_t *adj_diff, const float *rays, uint32_t num_rays, const uint32_t *start_point,
                  uint32_t num_quantiles, const float *depth_quantiles, float weight_threshold,
                  uint32_t max_intersections, void *rgba, float *depth, uint32_t *depth_idx, void *contribution,
                  uint32_t *num_intersections, float *distortion, float *W_total, float *S_total, float *t_far,
                  or_ray_stats *stats, int num_threads)
{
    int nt = set_threads(num_threads);
    uint32_t K = depth_quantiles ? num_quantiles : 0;
#pragma omp parallel for schedule(dynamic, 64) num_threads(nt)
    for (int64_t ri = 0; ri < (int64_t)num_rays; ++ri) {
        uint32_t r = (uint32_t)ri;
        fwd_state s;
        walk_dbg_t g;
        init_dbg(&g, NULL, 0);
        read_ray(rays, r, &s.o, &s.d);
        s.density = density;
        s.dm.kind = attr_f16 ? 1 : 0;
        s.dm.base = diffuse;
        s.dm.R = diff_res;
        s.sm.kind = attr_f16 ? 1 : 0;
        s.sm.base = specular;
        s.sm.R = spec_res;
        spec_setup(s.d, spec_res, &s.spec);
        s.thr = weight_threshold;
        s.f16 = attr_f16;
        s.contribution = contribution;
        s.qthr = K ? depth_quantiles + (size_t)r * K : NULL;
        s.nq = K;
        s.qi = 0;
        s.qval = K ? s.qthr[0] : 0.0f;
        s.qdepth = K ? depth + (size_t)r * K : NULL;
        s.qidx = K ? depth_idx + (size_t)r * K : NULL;
        s.acc = mk(0.0f, 0.0f, 0.0f);
        s.T = 1.0f;
        s.W = s.S = s.D = s.self = s.tfar = 0.0f;
        s.g = &g;
        uint32_t n =
            walk(s.o, s.d, points, adjacency, offsets, adj_diff, start_point[r], max_intersections, fwd_integrate, &s, &g);
        for (uint32_t i = s.qi; i < K; ++i) {
            depth[(size_t)r * K + i] = -1.0f;
            depth_idx[(size_t)r * K + i] = OR_NONE;
        }
        attr_store(attr_f16, rgba, 4 * (size_t)r + 0, s.acc.x);
        attr_store(attr_f16, rgba, 4 * (size_t)r + 1, s.acc.y);
        attr_store(attr_f16, rgba, 4 * (size_t)r + 2, s.acc.z);
        attr_store(attr_f16, rgba, 4 * (size_t)r + 3, 1.0f - s.T);
        if (num_intersections)
            num_intersections[r] = n;
        distortion[r] = fmaf(2.0f, s.D, s.self / 3.0f);
        W_total[r] = s.W;
        S_total[r] = s.S;
        t_far[r] = s.tfar;
        if (stats)
            stats[r] = g.st;
    }
}

/* ------------------------------------------------------------------------- */
/* training backward (ray_integrator_octmap.cuh:683-860, :979-1026)           */
/* ------------------------------------------------------------------------- */

/* ray_integrator.cuh:39-53 */
static inline v3 cell_intersection_grad(v3 prim, v3 opp, v3 o, v3 d)
{
    v3 fo = mk((prim.x + opp.x) * 0.5f, (prim.y + opp.y) * 0.5f, (prim.z + opp.z) * 0.5f);
    v3 n = vsub(opp, prim);
    float num = vdot(vsub(fo, o), n);
    float dp = vdot(n, d);
    v3 op = vsub(o, prim);
    v3 g = mk(fmaf(num, d.x, dp * op.x), fmaf(num, d.y, dp * op.y), fmaf(num, d.z, dp * op.z));
    return vdivs(g, dp * dp);
}

typedef struct {
    v3 o, d;
    const float *density;
    texmap_t dm, sm;
    bil_t spec;
    float thr;
    int f16;
    v3 acc;
    float T;
    float cur_depth_grad;
    uint32_t qi, nq;
    float qval;
    const float *qthr, *depth_grad;
    float *points_grad;
    void *diffuse_grad, *specular_grad, *point_error;
    float *density_grad;
    v3 prev_geom, prev_grad, cur_grad, next_grad;
    uint32_t prev_idx;
    v3 fwd_rgb, fwd_rgb_grad;
    float fwd_alpha, fwd_alpha_grad, ray_error;
    float W_run, S_run, W_total, S_total, dist_grad, D_total, D_running;
    walk_dbg_t *g;
} bwd_state;

static inline void add_vec_atomic(float *pg, uint32_t idx, v3 v)
{
    atomic_add_f32(pg + 3 * (size_t)idx + 0, v.x);
    atomic_add_f32(pg + 3 * (size_t)idx + 1, v.y);
    atomic_add_f32(pg + 3 * (size_t)idx + 2, v.z);
}

static int bwd_integrate(void *sp, uint32_t cell, float t0, float t1, v3 p, v3 np)
{
    bwd_state *s = (bwd_state *)sp;
    float sig = s->density[cell];
    v3 rgb = mk(0.0f, 0.0f, 0.0f);
    bil_t db;
    int has_color = 0;
    if (sig > 1e-6f) {
        s->g->st.shaded += 1;
        rgb = cell_color(&s->dm, &s->sm, &s->spec, cell, s->o, s->d, t0, p, &db);
        has_color = 1;
    }
    float dt = fmaxf(t1 - t0, 0.0f);
    float alpha = 1.0f - or_expf(-sig * dt);
    float w = s->T * alpha;
    float da_ds = dt * (1.0f - alpha);
    float da_ddt = 0.0f;
    if (dt > 0.0f)
        da_ddt = sig * (1.0f - alpha);

    s->acc = vfma(w, rgb, s->acc);
    if (s->point_error)
        attr_atomic_add(s->f16, s->point_error, cell, (g_plant == OR_PLANT_POINT_ERROR_ALPHA ? alpha : w) * s->ray_error);

    v3 dL_drgb = mk(s->fwd_rgb_grad.x * w, s->fwd_rgb_grad.y * w, s->fwd_rgb_grad.z * w);
    v3 rest = vsub(s->fwd_rgb, s->acc);
    rest = vdivs(rest, s->T * ((1.0f - alpha) + 1e-6f));
    float dL_dalpha = s->T * vdot(vsub(rgb, rest), s->fwd_rgb_grad);
    dL_dalpha = dL_dalpha + ((1.0f - s->fwd_alpha) * s->fwd_alpha_grad) / ((1.0f - alpha) + 1e-6f);

    float dL_ds = dL_dalpha * da_ds;
    float dL_ddt = dL_dalpha * da_ddt;
    float dL_dt0 = 0.0f;

    if (s->dist_grad != 0.0f) {
        float s0 = 1.0f - 1.0f / (1.0f + t0);
        float s1 = 1.0f - 1.0f / (1.0f + t1);
        float mid = 0.5f * (s0 + s1);
        float ds = s1 - s0;
        float Wm = s->W_run;
        float Sm = s->S_run;
        float Wp = (s->W_total - Wm) - w;
        float Sp = fmaf(-w, mid, s->S_total - Sm);
        float dL_dw_raw = fmaf(2.0f / 3.0f * w, ds, fmaf(2.0f, fmaf(-mid, Wp, Sp), 2.0f * fmaf(mid, Wm, -Sm)));
        float dL_dw_outer = dL_dw_raw * s->dist_grad;
        float dL_dw_w = dL_dw_outer * w;
        float D_iplus = (s->D_total - s->D_running) - dL_dw_w;
        dL_ds = dL_ds + fmaf(-dt, D_iplus, (dL_dw_outer * s->T) * da_ds);
        s->D_running = s->D_running + dL_dw_w;
        s->W_run = s->W_run + w;
        s->S_run = fmaf(w, mid, s->S_run);
    }

    float nextT = s->T * (1.0f - alpha);
    while (s->qi < s->nq && nextT < s->qval) {
        float dg = s->depth_grad[s->qi] / sig;
        dL_dt0 = dL_dt0 + dg;
        dL_ds = dL_ds + (-dg * or_logf(s->T / s->qval)) / sig;
        s->cur_depth_grad = s->cur_depth_grad - dg;
        s->qi++;
        if (s->qi < s->nq)
            s->qval = s->qthr[s->qi];
    }
    if (s->qi < s->nq) {
        dL_ds = fmaf(-dt, s->cur_depth_grad, dL_ds);
        dL_ddt = fmaf(-sig, s->cur_depth_grad, dL_ddt);
    }
    dL_dt0 = dL_dt0 + -dL_ddt;
    float dL_dt1 = dL_ddt;

    v3 dt0_dprev = mk(0.0f, 0.0f, 0.0f);
    if (s->prev_idx != OR_NONE && g_plant != OR_PLANT_NO_DT0_PREV)
        dt0_dprev = cell_intersection_grad(s->prev_geom, p, s->o, s->d);
    v3 dt1_dcur = cell_intersection_grad(p, np, s->o, s->d);
    v3 dt0_dcur = cell_intersection_grad(p, s->prev_geom, s->o, s->d);
    if (g_plant == OR_PLANT_NO_FIRST_CELL_TERM && s->prev_idx == OR_NONE)
        dt0_dcur = mk(0.0f, 0.0f, 0.0f);
    v3 dt1_dnext = cell_intersection_grad(np, p, s->o, s->d);

    s->prev_grad = vfma(dL_dt0, dt0_dprev, s->prev_grad);
    v3 cg = mk(fmaf(dL_dt1, dt1_dcur.x, dL_dt0 * dt0_dcur.x), fmaf(dL_dt1, dt1_dcur.y, dL_dt0 * dt0_dcur.y),
               fmaf(dL_dt1, dt1_dcur.z, dL_dt0 * dt0_dcur.z));
    s->cur_grad = vadd(s->cur_grad, cg);
    s->next_grad = vfma(dL_dt1, dt1_dnext, s->next_grad);

    if (s->prev_idx != OR_NONE)
        add_vec_atomic(s->points_grad, s->prev_idx, s->prev_grad);
    s->prev_geom = p;
    s->prev_idx = cell;
    s->prev_grad = s->cur_grad;
    s->cur_grad = s->next_grad;
    s->next_grad = mk(0.0f, 0.0f, 0.0f);

    s->T = nextT;

    if (has_color) {
        float gl[3];
        gl[0] = (dL_drgb.x * rgb.x) * (1.0f - rgb.x);
        gl[1] = (dL_drgb.y * rgb.y) * (1.0f - rgb.y);
        gl[2] = (dL_drgb.z * rgb.z) * (1.0f - rgb.z);
        size_t RRd = 3 * (size_t)s->dm.R * (size_t)s->dm.R;
        size_t RRs = 3 * (size_t)s->sm.R * (size_t)s->sm.R;
        size_t bd = (size_t)cell * RRd, bs = (size_t)cell * RRs;
        for (int c = 0; c < 3; ++c) {
            attr_atomic_add(s->f16, s->diffuse_grad, bd + (size_t)db.i00 * 3 + c, db.w00 * gl[c]);
            attr_atomic_add(s->f16, s->diffuse_grad, bd + (size_t)db.i10 * 3 + c, db.w10 * gl[c]);
            attr_atomic_add(s->f16, s->diffuse_grad, bd + (size_t)db.i01 * 3 + c, db.w01 * gl[c]);
            attr_atomic_add(s->f16, s->diffuse_grad, bd + (size_t)db.i11 * 3 + c, db.w11 * gl[c]);
        }
        for (int c = 0; c < 3; ++c) {
            attr_atomic_add(s->f16, s->specular_grad, bs + (size_t)s->spec.i00 * 3 + c, s->spec.w00 * gl[c]);
            attr_atomic_add(s->f16, s->specular_grad, bs + (size_t)s->spec.i10 * 3 + c, s->spec.w10 * gl[c]);
            attr_atomic_add(s->f16, s->specular_grad, bs + (size_t)s->spec.i01 * 3 + c, s->spec.w01 * gl[c]);
            attr_atomic_add(s->f16, s->specular_grad, bs + (size_t)s->spec.i11 * 3 + c, s->spec.w11 * gl[c]);
        }
    }
    atomic_add_f32(s->density_grad + cell, dL_ds);

    if (s->T < s->thr) {
        add_vec_atomic(s->points_grad, s->prev_idx, s->prev_grad);
        if (g_plant == OR_PLANT_FLUSH_CUR_ON_STOP)
            add_vec_atomic(s->points_grad, s->g->next, s->cur_grad);
        return 0;
    }
    return 1;
}

void or_trace_bwd(int attr_f16, const float *points, const void *diffuse, const void *specular, int diff_res,
                  int spec_res, const float *density, const uint32_t *adjacency, const uint32_t *offsets,
                  const uint16_t *adj_diff, const float *rays, uint32_t num_rays, const uint32_t *start_point,
                  const void *rgba, const void *rgba_grad, uint32_t num_quantiles, const float *depth_quantiles,
                  const uint32_t *depth_idx, const float *depth_grad, const void *ray_error,
                  float contribution_alpha_grad, const float *distortion, const float *distortion_grad,
                  const float *W_total, const float *S_total, const float *t_far, float weight_threshold,
                  uint32_t max_intersections, float *points_grad, void *diffuse_grad, void *specular_grad,
                  float *density_grad, void *point_error, or_ray_stats *stats, int num_threads)
{
    int nt = set_threads(num_threads);
    uint32_t K = depth_quantiles ? num_quantiles : 0;
    (void)t_far;
#pragma omp parallel for schedule(dynamic, 64) num_threads(nt)
    for (int64_t ri = 0; ri < (int64_t)num_rays; ++ri) {
        uint32_t r = (uint32_t)ri;
        bwd_state s;
        walk_dbg_t g;
        init_dbg(&g, NULL, 0);
        read_ray(rays, r, &s.o, &s.d);
        s.density = density;
        s.dm.kind = attr_f16 ? 1 : 0;
        s.dm.base = diffuse;
        s.dm.R = diff_res;
        s.sm.kind = attr_f16 ? 1 : 0;
        s.sm.base = specular;
        s.sm.R = spec_res;
        spec_setup(s.d, spec_res, &s.spec);
        s.thr = weight_threshold;
        s.f16 = attr_f16;
        float rg[4], rv[4];
        for (int i = 0; i < 4; ++i) {
            rg[i] = attr_load(attr_f16, rgba_grad, 4 * (size_t)r + i);
            rv[i] = attr_load(attr_f16, rgba, 4 * (size_t)r + i);
        }
        if (g_plant != OR_PLANT_IGNORE_CONTRIB_GRAD)
            rg[3] = rg[3] + contribution_alpha_grad;
        s.ray_error = ray_error ? attr_load(attr_f16, ray_error, r) : 0.0f;
        float cdg = 0.0f;
        for (uint32_t i = 0; i < K; ++i) {
            uint32_t qi = depth_idx[(size_t)r * K + i];
            if (qi != OR_NONE)
                cdg = cdg + depth_grad[(size_t)r * K + i] / density[qi];
        }
        s.acc = mk(0.0f, 0.0f, 0.0f);
        s.T = 1.0f;
        s.cur_depth_grad = cdg;
        s.qi = 0;
        s.nq = K;
        s.qthr = K ? depth_quantiles + (size_t)r * K : NULL;
        s.depth_grad = K ? depth_grad + (size_t)r * K : NULL;
        s.qval = K ? s.qthr[0] : 0.0f;
        s.points_grad = points_grad;
        s.diffuse_grad = diffuse_grad;
        s.specular_grad = specular_grad;
        s.density_grad = density_grad;
        s.point_error = point_error;
        s.prev_geom = s.prev_grad = s.cur_grad = s.next_grad = mk(0.0f, 0.0f, 0.0f);
        s.prev_idx = OR_NONE;
        s.fwd_rgb = mk(rv[0], rv[1], rv[2]);
        s.fwd_alpha = rv[3];
        s.fwd_rgb_grad = mk(rg[0], rg[1], rg[2]);
        s.fwd_alpha_grad = rg[3];
        s.W_run = s.S_run = s.D_running = 0.0f;
        s.W_total = W_total ? W_total[r] : 0.0f;
        s.S_total = S_total ? S_total[r] : 0.0f;
        float fd = distortion ? distortion[r] : 0.0f;
        s.dist_grad = distortion_grad ? distortion_grad[r] : 0.0f;
        s.D_total = (2.0f * fd) * s.dist_grad;
        s.g = &g;
        walk(s.o, s.d, points, adjacency, offsets, adj_diff, start_point[r], max_intersections, bwd_integrate, &s, &g);
        if (stats)
            stats[r] = g.st;
    }
}

/* ------------------------------------------------------------------------- */
/* nearest site (what NNBVH.query returns, nn_bvh.cu:29-41), brute force      */
/* ------------------------------------------------------------------------- */

/* Exact nearest site of each query: squared distance dot(q-p, q-p) in fp32
 * with the dot convention above, ties -> lowest index. */
void or_nearest_site(const float *points, uint32_t num_points, const float *queries, uint32_t num_queries,
                     int32_t *out, int num_threads)
{
    int nt = set_threads(num_threads);
#pragma omp parallel for schedule(dynamic, 16) num_threads(nt)
    for (int64_t qi = 0; qi < (int64_t)num_queries; ++qi) {
        v3 q = ld3(queries, (uint32_t)qi);
        float best = INFINITY;
        int32_t bi = -1;
        for (uint32_t i = 0; i < num_points; ++i) {
            v3 df = vsub(q, ld3(points, i));
            float d2 = vdot(df, df);
            if (d2 < best) {
                best = d2;
                bi = (int32_t)i;
            }
        }
        out[qi] = bi;
    }
}

/* exported for tests: ray_integrator.cuh:39-53 */
void or_cell_intersection_grad(const float prim[3], const float opp[3], const float o[3], const float d[3],
                               float out[3])
{
    v3 g = cell_intersection_grad(mk(prim[0], prim[1], prim[2]), mk(opp[0], opp[1], opp[2]), mk(o[0], o[1], o[2]),
                                  mk(d[0], d[1], d[2]));
    out[0] = g.x;
    out[1] = g.y;
    out[2] = g.z;
}

/* ------------------------------------------------------------------------- */
/* camera rays                                                                 */
/* ------------------------------------------------------------------------- */

/* sin x and cos x for x in [0, pi]: reduced to [-pi/4, pi/4] against pi/2
 * or pi, each held as hi + lo (hi - x is exact there by Sterbenz's lemma,
 * so the reduced argument is rounded once), then the Taylor polynomials of
 * degree 13 (sin) and 14 (cos) in Horner form in z = r^2 (truncation below
 * 3e-14 on [-pi/4, pi/4]).  Same operations as vt_sinf / vt_cosf. */
#define OR_PI_HI 0x1.921fb6p+1f
#define OR_PI_LO (-0x1.777a5cp-24f)
#define OR_PIO2_HI 0x1.921fb6p+0f
#define OR_PIO2_LO (-0x1.777a5cp-25f)
#define OR_PIO4 0.785398185f
#define OR_PI3O4 2.35619450f

static inline float sin_poly(float r)
{
    const float z = r * r;
    float p = 1.0f / 6227020800.0f;
    p = fmaf(p, z, -1.0f / 39916800.0f);
    p = fmaf(p, z, 1.0f / 362880.0f);
    p = fmaf(p, z, -1.0f / 5040.0f);
    p = fmaf(p, z, 1.0f / 120.0f);
    p = fmaf(p, z, -1.0f / 6.0f);
    return fmaf(r * z, p, r);
}

static inline float cos_poly(float r)
{
    const float z = r * r;
    float p = -1.0f / 87178291200.0f;
    p = fmaf(p, z, 1.0f / 479001600.0f);
    p = fmaf(p, z, -1.0f / 3628800.0f);
    p = fmaf(p, z, 1.0f / 40320.0f);
    p = fmaf(p, z, -1.0f / 720.0f);
    p = fmaf(p, z, 1.0f / 24.0f);
    p = fmaf(p, z, -0.5f);
    return fmaf(z, p, 1.0f);
}

float or_sinf(float x)
{
    if (x <= OR_PIO4)
        return sin_poly(x);
    if (x <= OR_PI3O4)
        return cos_poly((OR_PIO2_HI - x) + OR_PIO2_LO); /* sin x = cos(pi/2 - x) */
    return sin_poly((OR_PI_HI - x) + OR_PI_LO);         /* sin x = sin(pi - x) */
}

float or_cosf(float x)
{
    if (x <= OR_PIO4)
        return cos_poly(x);
    if (x <= OR_PI3O4)
        return sin_poly((OR_PIO2_HI - x) + OR_PIO2_LO); /* cos x = sin(pi/2 - x) */
    return -cos_poly((OR_PI_HI - x) + OR_PI_LO);        /* cos x = -cos(pi - x) */
}

void or_sincos_many(int cos, const float *x, float *y, size_t n)
{
    for (size_t i = 0; i < n; ++i)
        y[i] = cos ? or_cosf(x[i]) : or_sinf(x[i]);
}

/* Pixel (u, v): normalised image coordinates (pixel centre at +pixel_offset,
 * datasets.py:128-131), through the camera model to a camera-frame
 * direction, normalised (datasets.py:133-134), rotated by the pose
 * (datasets.py:296-299), origin t (+ the rolling-shutter shift of row v). */
static void camera_ray(const or_camera *c, uint32_t u, uint32_t v, uint32_t H, float *q)
{
    const float mx = ((float)u + c->pixel_offset - c->cx) / c->fx;
    const float my = ((float)v + c->pixel_offset - c->cy) / c->fy;
    v3 dc = mk(mx, my, 1.0f);
    if (c->model == OR_CAMERA_FISHEYE) {
        const float td = sqrtf(fmaf(my, my, mx * mx));
        dc = mk(0.0f, 0.0f, 1.0f);
        if (td > 0.0f) {
            /* Newton on theta (1 + k1 theta^2 + k2 theta^4 + k3 theta^6 + k4 theta^8) = td */
            float th = td;
            for (int it = 0; it < 12; ++it) {
                const float t2 = th * th;
                const float p = fmaf(fmaf(fmaf(c->k[3], t2, c->k[2]), t2, c->k[1]), t2, c->k[0]);
                const float qq =
                    fmaf(fmaf(fmaf(9.0f * c->k[3], t2, 7.0f * c->k[2]), t2, 5.0f * c->k[1]), t2, 3.0f * c->k[0]);
                const float g = fmaf(th * t2, p, th) - td;
                const float dg = fmaf(t2, qq, 1.0f);
                th = th - g / dg;
            }
            th = fminf(fmaxf(th, 0.0f), OR_PI_HI);
            const float s = or_sinf(th) / td;
            dc = mk(mx * s, my * s, or_cosf(th));
        }
    }
    dc = vdivs(dc, sqrtf(vdot(dc, dc)));
    const v3 d = mk(vdot(mk(c->R[0], c->R[1], c->R[2]), dc), vdot(mk(c->R[3], c->R[4], c->R[5]), dc),
                    vdot(mk(c->R[6], c->R[7], c->R[8]), dc));
    const float sv = H > 1 ? (float)v / (float)(H - 1) : 0.0f;
    q[0] = fmaf(sv, c->rolling[0], c->t[0]);
    q[1] = fmaf(sv, c->rolling[1], c->t[1]);
    q[2] = fmaf(sv, c->rolling[2], c->t[2]);
    q[3] = d.x;
    q[4] = d.y;
    q[5] = d.z;
}

void or_camera_rays(const or_camera *cams, uint32_t num_images, uint32_t H, uint32_t W, float *rays)
{
    for (uint32_t img = 0; img < num_images; ++img)
        for (uint32_t v = 0; v < H; ++v)
            for (uint32_t u = 0; u < W; ++u)
                camera_ray(&cams[img], u, v, H, rays + 6 * (((size_t)img * H + v) * W + u));
}
