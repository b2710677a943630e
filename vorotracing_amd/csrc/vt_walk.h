// vt_walk.h -- the Voronoi cell walk (tracing_octmap.cu:39-123) and the
// lane -> ray mapping of the traversal launches.
#pragma once

#include "vt_device.h"

namespace vt {

// Exit-face order without a division per face.  For dp, bdp > 0,
// num/dp < bnum/bdp <=> A < B with A = num*bdp, B = bnum*dp.  The search
// forms Q = RN(B), gap = RN(A - Q) (one fma) and h = RN(|Q| - 2^18 |gap|)
// (one fma).  When h < -c (c = 1e-26f; rounding is monotone, so then
// 2^18 |gap| > |Q| + c exactly):
//  - Q is off B by at most max(2^-24 |Q|, 2^-150) and gap off A - Q by
//    2^-24 |gap|, both far below |gap| > 2^-18 (|Q| + c), so A - B has the
//    sign of gap;
//  - |A - B| >= 0.98 * 2^-18 (|Q| + c), so the quotients x = num/dp and
//    y = bnum/bdp differ by at least 2^-19 |y| and, as dp, bdp <= |f16
//    offset| < 2^17, by at least 2^-18 c / 2^34 > 2^-138.  Two reals that
//    far apart cannot round to the same finite float (one normal rounding
//    moves 2^-24 relative, a subnormal one 2^-150), so RN(x) < RN(y) iff
//    gap < 0.  Overflow cannot turn an accept into a tie: the largest best
//    is 2^128 (below), and x <= 2^128 (1 - 2^-19) rounds to a finite float.
// Every other case (near-ties, overflow, NaN: h is then NaN or >= -c)
// compares the two IEEE quotients, so the choice is the reference's
// RN(num/dp) < RN(bnum/bdp), bit for bit, provided RN(bnum/bdp) > -inf:
// below -2^128 two quotients that differ by 2^-19 both round to -inf and the
// reference keeps the first, so exit_face redoes such a search with IEEE
// quotients.  Before the first candidate the best is the pair (2^64, 2^-64):
// its quotient 2^128 rounds to +inf, which is the reference's initial t_1,
// and the same test then accepts a face iff RN(num/dp) < inf.
constexpr float FIRST_BNUM = 0x1p64f;
constexpr float FIRST_BDP = 0x1p-64f;

__device__ __forceinline__ bool exit_before(float num, float dp, float bnum, float bdp)
{
    float Q = bnum * dp;
    float gap = fma_(num, bdp, -Q);
    // false for NaN and for |Q| = inf, which therefore need no test of their own
    float h = fma_(__builtin_fabsf(gap), -0x1p18f, __builtin_fabsf(Q));
    if (h < -1e-26f)
        return gap < 0.0f;
    return num / dp < bnum / bdp;
}

// f16 halves of a packed face record (x | y << 16, z | w << 16), widened
// exactly.
__device__ __forceinline__ float half_lo(uint32_t w) { return h2f((uint16_t)(w & 0xffffu)); }
__device__ __forceinline__ float half_hi(uint32_t w) { return h2f((uint16_t)(w >> 16)); }

// f16 face record -> offset (ox, oy, oz) and the plane terms of the walk:
// dp = off . d and num = (p + off/2 - o) . off.
__device__ __forceinline__ void face_terms(uint2 r, f3 p, f3 o, f3 d, float &num, float &dp)
{
    const float ox = half_lo(r.x), oy = half_hi(r.x), oz = half_lo(r.y);
    dp = fma_(oz, d.z, fma_(oy, d.y, ox * d.x));
    const float ex = fma_(ox, 0.5f, p.x) - o.x;
    const float ey = fma_(oy, 0.5f, p.y) - o.y;
    const float ez = fma_(oz, 0.5f, p.z) - o.z;
    num = fma_(ez, oz, fma_(ey, oy, ex * ox));
}

// The exit face of a cell whose face records are fl[0, nf): the lowest index
// j with dp_j > 0 minimising RN(num_j / dp_j) (tracing_octmap.cu:73-100), and
// t1 = that quotient.  NONE when no face has dp > 0 (t1 is then not set).
// Faces are read in chunks of CHUNK records; records past the list end stay
// inside the 32-row padding and are masked, so the choice does not depend on
// CHUNK.
template <int CHUNK>
__device__ __forceinline__ uint32_t exit_face(const uint2 *fl, uint32_t nf, f3 p, f3 o, f3 d, float &t1)
{
    // The running minimum is kept as the pair (bnum, bdp) and candidates are
    // ordered by exit_before.
    static_assert(CHUNK >= 1 && CHUNK <= 32, "reads past a list end must stay inside the 32-row padding");
    uint32_t best = NONE;
    float bnum = FIRST_BNUM, bdp = FIRST_BDP;
    for (uint32_t i = 0; i < nf; i += CHUNK) {
        uint2 rec[CHUNK];
#pragma unroll
        for (int j = 0; j < CHUNK; ++j)
            rec[j] = fl[i + j];
#pragma unroll
        for (int j = 0; j < CHUNK; ++j) {
            // Widen the halves once (v_cvt_f32_f16) and share them between
            // dp and num: the empty asm keeps the compiler from folding the
            // widening into v_fma_mix_f32 operands, which issue at a lower
            // rate than a conversion plus plain fmas.
            float ox = half_lo(rec[j].x), oy = half_hi(rec[j].x), oz = half_lo(rec[j].y);
            asm("" : "+v"(ox), "+v"(oy), "+v"(oz));
            float dp = fma_(oz, d.z, fma_(oy, d.y, ox * d.x));
            if (dp > 0.0f && (i + j) < nf) {
                // p + off/2: off/2 is exact, so the fma rounds once like p + off*0.5
                float ex = fma_(ox, 0.5f, p.x) - o.x;
                float ey = fma_(oy, 0.5f, p.y) - o.y;
                float ez = fma_(oz, 0.5f, p.z) - o.z;
                float num = fma_(ez, oz, fma_(ey, oy, ex * ox));
                if (exit_before(num, dp, bnum, bdp)) {
                    bnum = num;
                    bdp = dp;
                    best = i + j;
                }
            }
        }
    }
    if (best == NONE)
        return NONE;
    t1 = bnum / bdp;
    if (t1 == -__builtin_huge_valf()) {
        // A quotient rounded to -inf: the reference keeps the first face that
        // reaches it, which exit_before cannot see (see above).  Redo the
        // search with IEEE quotients.
        float bt = __builtin_huge_valf();
        best = NONE;
        for (uint32_t j = 0; j < nf; ++j) {
            float num, dp;
            face_terms(fl[j], p, o, d, num, dp);
            if (dp > 0.0f) {
                const float t = num / dp;
                if (t < bt) {
                    bt = t;
                    best = j;
                }
            }
        }
        t1 = bt;
    }
    return best;
}

// State of one walk between steps: current cell and site, entry distance
// t0, and the step count n of trace_octmap (tracing_octmap.cu:50-54); plus
// the current cell's face-list range [b, e), loaded with its site so that a
// step starts with one dependent load fewer.
struct WalkState {
    uint32_t cur;
    f3 p;
    float t0;
    uint32_t n;
    uint32_t b, e;
};

__device__ __forceinline__ void walk_begin(WalkState &w, const float *points, const uint32_t *offsets,
                                           uint32_t start)
{
    w.cur = start;
    w.p = load_site(points, start);
    w.b = offsets[start];
    w.e = offsets[start + 1];
    w.t0 = 0.0f;
    w.n = 0;
}

// One iteration of the cell walk (tracing_octmap.cu:56-120): searches the
// current cell's face list for the nearest bisector plane with n.d > 0
// (lowest face index wins ties), hands [t0, t1) to the integrator when
// t1 > t0, and moves to the neighbour behind that face.  Returns false when
// the walk ends (step cap, no exit face, or the integrator stops it); w.n is
// then the reference's return value.  The integrator's
// begin_cell(cur) runs before the face search, so that loads it issues
// (the cell's density) overlap the search.
template <int CHUNK, class Integrator, class StatsT>
__device__ __forceinline__ bool walk_step(WalkState &w, f3 o, f3 d, const float *points,
                                          const uint32_t *adjacency,
                                          const uint32_t *offsets, const uint2 *adj_diff,
                                          uint32_t max_steps, Integrator &integ, StatsT &st)
{
    w.n++;
    if (w.n > max_steps)
        return false;
    const f3 p = w.p;
    const uint32_t b = w.b;
    const uint32_t nf = w.e - b;
    integ.begin_cell(w.cur); // the integrator's own loads for the cell, issued before the face loop
    st.visit(w.cur, nf);
    float t1;
    const uint32_t best = exit_face<CHUNK>(adj_diff + b, nf, p, o, d, t1);
    if (best == NONE)
        return false;
    st.exit();
    uint32_t nxt = adjacency[b + best];
    f3 np = load_site(points, nxt);
    const uint32_t nb = offsets[nxt], ne = offsets[nxt + 1];
    // No early return inside the integrate branch: a divergent exit there made
    // the control flow unstructured, and hipcc (packed FP32 disabled) then
    // reused np's registers inside the shading code while np was still live,
    // corrupting the next site of integrating lanes.  The state update below
    // is harmless when the integrator ends the walk.
    bool go = true;
    if (t1 > w.t0) {
        st.integrate();
        go = integ.integrate(w.cur, w.t0, t1, p, np, st);
    }
    w.t0 = __builtin_fmaxf(w.t0, t1);
    w.cur = nxt;
    w.p = np;
    w.b = nb;
    w.e = ne;
    return go;
}

// The whole walk of one ray (trace_octmap, tracing_octmap.cu:39-123).
// Returns the reference's step count n (the breaking iteration included).
template <int CHUNK, class Integrator, class StatsT>
__device__ __forceinline__ uint32_t walk(f3 o, f3 d, const float *points,
                                         const uint32_t *adjacency,
                                         const uint32_t *offsets, const uint2 *adj_diff,
                                         uint32_t start, uint32_t max_steps, Integrator &integ, StatsT &st)
{
    WalkState w;
    walk_begin(w, points, offsets, start);
    while (walk_step<CHUNK>(w, o, d, points, adjacency, offsets, adj_diff, max_steps, integ, st)) {
    }
    return w.n;
}

// ---------------------------------------------------------------------------
// The same walk over the packed walk layout (vt_walk_layout, built by
// vt_walk_layout_fill).  The traversal kernels are bound by the number of
// vector memory instructions they issue, so the layout regroups the scene's
// arrays to need fewer of them per step:
//  - chunks: a cell's face records in chunks of 8, 16-byte aligned, each
//    face's x, y, z halves in turn (48 bytes, three uint4 rows): three loads
//    per 8 faces instead of four, and no per-face bound test, since a list is
//    padded to a multiple of 8 with zero offsets (n.d = 0 is never an exit
//    face);
//  - links: per padded face slot, the neighbour behind it with its own chunk
//    range, so the next cell's face records can be loaded as soon as the exit
//    face is known, in parallel with its site;
//  - cells: site and density in one 16-byte record;
//  - a cell's faces may be reordered (vt_walk_layout_fill's face order: by one
//    component of their offsets, so that the lanes of a wave, whose rays point
//    alike, meet forward-facing faces at the same slots and the wave skips the
//    plane test of slots that no lane faces); orig[slot] keeps each slot's
//    index in the original list for the exact-tie rule (exit_before_tie).
// A step reads the same offsets, sites and densities as walk_step, so it
// picks the same exit faces and hands the integrator the same values.
constexpr uint32_t WL_ID_BITS = 24;
constexpr uint32_t WL_ID_MASK = (1u << WL_ID_BITS) - 1u;
constexpr uint32_t WL_MAX_CHUNKS = 255; // chunks of one cell (8 bits beside the id)

struct PackedWalk {
    uint32_t cur; // cell
    uint32_t nch; // chunks of its face list
    uint32_t cb;  // its first chunk
    f3 p;
    float dens;
    float t0;
    uint32_t n;
    uint4 r0; // the first row of its first chunk (faces 0-1), loaded with its site
};

// The first row of a cell's first chunk (the chunk array holds one chunk
// past its last, so an empty list reads in bounds too).
__device__ __forceinline__ void load_first_chunk(PackedWalk &w, const uint4 *chunks)
{
    w.r0 = chunks[3 * (size_t)w.cb];
}

__device__ __forceinline__ void walk_begin_packed(PackedWalk &w, const uint2 *heads, const float4 *cells,
                                                  const uint4 *chunks, uint32_t start)
{
    const uint2 h = heads[start];
    const float4 c = cells[start];
    w.cur = start;
    w.nch = h.x >> WL_ID_BITS;
    w.cb = h.y;
    w.p = mk(c.x, c.y, c.z);
    w.dens = c.w;
    w.t0 = 0.0f;
    w.n = 0;
    load_first_chunk(w, chunks);
}

__device__ __forceinline__ uint32_t chunk_word(uint4 r0, uint4 r1, uint4 r2, int k)
{
    const uint4 r = k < 4 ? r0 : k < 8 ? r1 : r2;
    k &= 3;
    return k == 0 ? r.x : k == 1 ? r.y : k == 2 ? r.z : r.w;
}

__device__ __forceinline__ float chunk_half(uint4 r0, uint4 r1, uint4 r2, int h)
{
    const uint32_t w = chunk_word(r0, r1, r2, h >> 1);
    return (h & 1) ? half_hi(w) : half_lo(w);
}

// Offset of face j (0..7) of a chunk whose 24 halves (x, y, z of face 0, then
// of face 1, ...) are the rows R0, R1, R2: faces 0-1 lie in R0, 2-4 end in
// R1 and 5-7 in R2, so the search starts as the first row arrives.
__device__ __forceinline__ void chunk_face(uint4 R0, uint4 R1, uint4 R2, int j, float &ox, float &oy, float &oz)
{
    ox = chunk_half(R0, R1, R2, 3 * j);
    oy = chunk_half(R0, R1, R2, 3 * j + 1);
    oz = chunk_half(R0, R1, R2, 3 * j + 2);
}

// exit_before for the packed layout, whose face lists may be reordered
// (vt_walk_layout_fill's face order): two quotients that round to the same
// float go to the face of lower index in the cell's original list, as the
// reference's strict t < t_1 over that list keeps the first
// (tracing_octmap.cu:90-94).  Such ties only occur on the IEEE path (a
// decided comparison separates the quotients by 2^-19 of their size, and two
// that both round to -inf take the -inf redo), where a tie with a face
// (bt < inf: only the virtual first best has quotient +inf) sets bnum to NaN.
// No later face is then accepted (a NaN quotient compares false), t1 comes
// out NaN, and the step settles the cell by exit_face_packed_ieee, which
// compares original indices.  A face's own quotient is never NaN when
// accepted, so NaN marks a tie and nothing else.
__device__ __forceinline__ bool exit_before_tie(float num, float dp, float &bnum, float bdp)
{
    float Q = bnum * dp;
    float gap = fma_(num, bdp, -Q);
    float h = fma_(__builtin_fabsf(gap), -0x1p18f, __builtin_fabsf(Q));
    if (h < -1e-26f)
        return gap < 0.0f;
    const float t = num / dp, bt = bnum / bdp;
    if (t == bt && bt < __builtin_huge_valf())
        bnum = __builtin_nanf("");
    return t < bt;
}

// The faces of one chunk (rows R0-R2, slots 8q..8q+7) against the running
// best (exit_face's order; an exact tie turns bnum into NaN); an accepted
// slot is kept as j - 16 (an inline constant, no move per face) and made
// 8q + j after the chunk.
__device__ __forceinline__ void search_chunk(uint4 R0, uint4 R1, uint4 R2, uint32_t q, f3 p, f3 o, f3 d,
                                             float &bnum, float &bdp, uint32_t &best)
{
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        float ox, oy, oz;
        chunk_face(R0, R1, R2, j, ox, oy, oz);
        // as in exit_face: keep the widening out of v_fma_mix operands
        asm("" : "+v"(ox), "+v"(oy), "+v"(oz));
        float dp = fma_(oz, d.z, fma_(oy, d.y, ox * d.x));
        if (dp > 0.0f) {
            float ex = fma_(ox, 0.5f, p.x) - o.x;
            float ey = fma_(oy, 0.5f, p.y) - o.y;
            float ez = fma_(oz, 0.5f, p.z) - o.z;
            float num = fma_(ez, oz, fma_(ey, oy, ex * ox));
            if (exit_before_tie(num, dp, bnum, bdp)) {
                bnum = num;
                bdp = dp;
                best = (uint32_t)(j - 16);
            }
        }
    }
    if ((int32_t)best < -8)
        best += 16 + 8 * q;
}

// The IEEE search over the nch chunks at ch, for a best quotient that rounded
// to -inf or an exact tie (t1 NaN): the lowest RN(num / dp), ties to the
// lowest orig[slot].  Returns the slot and sets t1.
__device__ __forceinline__ uint32_t exit_face_packed_ieee(const uint4 *ch, uint32_t nch, f3 p, f3 o, f3 d,
                                                          const uint16_t *orig, float &t1)
{
    float bt = __builtin_huge_valf();
    uint32_t best = NONE;
    for (uint32_t q = 0; q < nch; ++q) {
        const uint4 R0 = ch[3 * q], R1 = ch[3 * q + 1], R2 = ch[3 * q + 2];
        for (int j = 0; j < 8; ++j) {
            float ox, oy, oz;
            chunk_face(R0, R1, R2, j, ox, oy, oz);
            const float dp = fma_(oz, d.z, fma_(oy, d.y, ox * d.x));
            if (dp > 0.0f) {
                const float ex = fma_(ox, 0.5f, p.x) - o.x;
                const float ey = fma_(oy, 0.5f, p.y) - o.y;
                const float ez = fma_(oz, 0.5f, p.z) - o.z;
                const float t = fma_(ez, oz, fma_(ey, oy, ex * ox)) / dp;
                const uint32_t slot = 8 * q + j;
                if (t < bt || (t == bt && best != NONE && orig[slot] < orig[best])) {
                    bt = t;
                    best = slot;
                }
            }
        }
    }
    t1 = bt;
    return best;
}

// walk_step over the packed layout, with the loads of the next cell moved
// ahead: the exit face's link is loaded before the exit distance is divided
// out, and the next cell's site, density and (PRELOAD) the first row of its
// first chunk as soon as the link arrives, so that their latency overlaps the
// integrator's work.  Without PRELOAD that row is loaded with the rest of the
// chunk (for integrators with too little register room to hold it).  The
// integrator takes the density from the walk state (begin_cell_value).
// Statistics that record face counts read them from offsets; otherwise a
// visit counts the cell's padded slots.
template <bool PRELOAD, class Integrator, class StatsT>
__device__ __forceinline__ bool walk_step_packed(PackedWalk &w, f3 o, f3 d, const uint4 *chunks, const uint2 *links,
                                                 const float4 *cells, const uint16_t *origs,
                                                 const uint32_t *offsets, uint32_t max_steps, Integrator &integ,
                                                 StatsT &st)
{
    w.n++;
    if (w.n > max_steps)
        return false;
    const f3 p = w.p;
    integ.begin_cell_value(w.dens);
    if constexpr (StatsT::EXACT_FACES)
        st.visit(w.cur, offsets[w.cur + 1] - offsets[w.cur]);
    else
        st.visit(w.cur, 8 * w.nch);
    const uint4 *ch = chunks + 3 * (size_t)w.cb;
    uint32_t best = NONE;
    float bnum = FIRST_BNUM, bdp = FIRST_BDP;
    if (w.nch > 0)
        search_chunk(PRELOAD ? w.r0 : ch[0], ch[1], ch[2], 0, p, o, d, bnum, bdp, best);
    for (uint32_t q = 1; q < w.nch; ++q) {
        const uint4 *c = ch + 3 * q;
        search_chunk(c[0], c[1], c[2], q, p, o, d, bnum, bdp, best);
    }
    if (best == NONE)
        return false;
    st.exit();
    uint2 lk = links[8 * (size_t)w.cb + best];
    float t1 = bnum / bdp;
    if (!(t1 > -__builtin_huge_valf())) { // -inf, or NaN after a tie
        best = exit_face_packed_ieee(ch, w.nch, p, o, d, origs + 8 * (size_t)w.cb, t1);
        lk = links[8 * (size_t)w.cb + best];
    }
    const uint32_t cur = w.cur;
    w.cur = lk.x & WL_ID_MASK;
    w.nch = lk.x >> WL_ID_BITS;
    w.cb = lk.y;
    const float4 c = cells[w.cur];
    if constexpr (PRELOAD)
        load_first_chunk(w, chunks);
    // no early return inside the integrate branch (see walk_step)
    bool go = true;
    if (t1 > w.t0) {
        st.integrate();
        go = integ.integrate(cur, w.t0, t1, p, mk(c.x, c.y, c.z), st);
    }
    // max(t0, t1) as a select: neither is NaN, and fmaxf would add two
    // canonicalising moves
    w.t0 = t1 > w.t0 ? t1 : w.t0;
    w.p = mk(c.x, c.y, c.z);
    w.dens = c.w;
    return go;
}

// Cost of a screen tile for the launch order of the next launch over the
// same rays (vt_tile_order): TILE_COST_STEP x the longest walk's steps + the
// most face records one ray of the tile searched, both maxima over the
// tile's rays (a wave takes about as long as its longest lane).  Of the keys
// tried on C3 frames this one ordered the launch best; walk steps alone
// recovered about half as much.
constexpr uint32_t TILE_COST_STEP = 18;

__device__ __forceinline__ uint32_t tile_cost_of(uint32_t steps_max, uint32_t faces_max)
{
    return TILE_COST_STEP * steps_max + faces_max;
}

// Screen tiles are visited in vertical strips TILE_STRIP tiles wide (the last
// strip takes the remainder), row by row inside a strip; 0 = row-major over
// the whole image.  Consecutive waves then cover a compact screen region
// rather than an image-wide band, and so do the runs of consecutive blocks
// that one XCD takes in turn (xcd_interleaved_block).
#ifndef VT_TILE_STRIP
#define VT_TILE_STRIP 4
#endif
constexpr uint32_t TILE_STRIP = VT_TILE_STRIP;

// Lane -> ray for a tiled image batch: one wave (64 lanes) per tile_w x
// tile_h screen tile, tiles in vertical strips STRIP tiles wide.  Returns
// NONE for lanes past the image edge.
template <uint32_t STRIP = TILE_STRIP>
__device__ __forceinline__ uint32_t tiled_ray(uint32_t lane_global, uint32_t num_images, uint32_t H, uint32_t W,
                                              uint32_t th, uint32_t tw)
{
    uint32_t tile = lane_global / (th * tw);
    uint32_t within = lane_global % (th * tw);
    uint32_t tiles_x = (W + tw - 1) / tw;
    uint32_t tiles_y = (H + th - 1) / th;
    uint32_t tpi = tiles_x * tiles_y;
    uint32_t img = tile / tpi;
    uint32_t ti = tile % tpi;
    uint32_t tx, ty;
    if (STRIP == 0 || STRIP >= tiles_x) {
        ty = ti / tiles_x;
        tx = ti % tiles_x;
    } else {
        uint32_t per_strip = STRIP * tiles_y;
        uint32_t strip = ti / per_strip;
        uint32_t r = ti % per_strip;
        uint32_t w = STRIP;
        if ((strip + 1) * STRIP > tiles_x)
            w = tiles_x - strip * STRIP;
        ty = r / w;
        tx = strip * STRIP + r % w;
    }
    uint32_t y = ty * th + within / tw;
    uint32_t x = tx * tw + within % tw;
    if (img >= num_images || x >= W || y >= H)
        return NONE;
    return (img * H + y) * W + x;
}

} // namespace vt
