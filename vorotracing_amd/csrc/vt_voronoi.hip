// vt_voronoi.hip -- Voronoi neighbours (the Delaunay adjacency CSR) of a site
// set, built on the GPU.  Replaces the adjacency step of
// vorotracing.cuda.build_voronoi_adjacency (cuda/__init__.py:16-46, which
// calls Paragram; the synthetic scenes of this build use host qhull).
//
// One wave per cell; the cell lives in LDS and is clipped in double
// precision, in site-local coordinates:
//   * it starts as a box around all sites (6 planes), 10^6 times their
//     extent, so that the faces between convex-hull sites (unbounded in the
//     Delaunay sense) keep a part inside it;
//   * sites are taken from a uniform grid in distance bands [rho/2, rho)
//     with rho doubling; a site q cuts the cell by its bisector plane
//     d.x <= |d|^2/2 (d = q - p, exact in double for f32 inputs) when some
//     vertex lies strictly outside it;
//   * the walk stops once 2R <= rho (R: largest vertex distance; no farther
//     site can cut the cell) or the bands have passed every site;
//   * the neighbours are the sites whose planes keep a face, ascending.
// The cell is kept as the triangulation of its dual (Ray, Sokolov, Lefebvre,
// Levy, "Meshless Voronoi on the GPU", 2018): a vertex is a triangle of three
// plane ids; a cut removes the vertices strictly outside the plane and closes
// the hole with triangles (u, v, new plane) along the boundary edges (u, v).
//
// The scan is spread over the 64 lanes and pruned at three levels:
//   * rows of grid cells: only the spherical shell of cells that can hold
//     sites of the band;
//   * grid cells (one per lane): skipped when no point x of the cell's box
//     can satisfy x.v > |x|^2/2 for a vertex v, bounding max x.v by the
//     bounding box of the near vertices and by each far (box) vertex;
//   * candidates (one per lane, packed across the surviving grid cells of a
//     row): the same test for the site itself, then the exact vertex test.
// The planes that cut are applied one at a time, each cut spread over the
// lanes.  A first pass runs every cell with small tables; the few cells that
// overflow them run again with large ones.
#include "vt_internal.h"
#include "vt_prims.h"

#include <algorithm>
#include <cmath>

namespace vt {

constexpr uint32_t VOR_NONE = 0xffffffffu;
constexpr int VOR_BLOCK = 64; // one wave

// Per-cell capacities.  Plane ids are bytes, so P <= 255.
template <int P_, int T_, int E_> struct VorCap {
    static constexpr int P = P_; // planes (6 box + bisectors), also bounds the neighbours
    static constexpr int T = T_; // vertices
    static constexpr int E = E_; // directed edges of the region removed by one cut
};
using VorSmall = VorCap<96, 192, 96>;
// The large tier's edge table holds the edges of every vertex at once, so a
// cut that removes most of a cell (a near site after many slivers of a dense
// layer farther away) never overflows it.
using VorLarge = VorCap<255, 510, 3 * 510>;
// Neighbour lists: LIST_K entries per site; longer lists in slots of BIG_K.
constexpr int LIST_K = 64;
constexpr int BIG_K = VorLarge::P;

struct VorGrid {
    float lo[3];
    float h;       // cell side
    uint32_t g[3]; // cells per axis
    double box_lo[3], box_hi[3];
    double far2;   // squared local distance beyond which a vertex counts as far
};

enum { VOR_OK = 0, VOR_FULL = 1, VOR_DEGENERATE = 2 };
// which table overflowed (bits of the fails[F_REASON] word)
enum { FULL_PLANES = 1, FULL_EDGES = 2, FULL_VERTICES = 4, FULL_LISTS = 8 };

// fails[] words: failures, the retry count, big-list slots, work counters
enum {
    F_FULL = 0,
    F_DEGENERATE = 1,
    F_RETRY = 2,
    F_BIG = 3,
    F_NEXT0 = 4,
    F_NEXT1 = 5,
    F_FIRST_BAD = 6,
    F_REASON = 7,
    F_WORDS = 8
};

__device__ __forceinline__ double4 cross_d(double4 a, double4 b)
{
    return make_double4(a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x, 0.0);
}
__device__ __forceinline__ double dot_d(double4 a, double4 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }

// intersection of three planes n.x <= w; w of the result = |v|^2
__device__ __forceinline__ double4 plane_vertex(double4 a, double4 b, double4 d)
{
    double4 bc = cross_d(b, d), ca = cross_d(d, a), ab = cross_d(a, b);
    double det = dot_d(a, bc);
    double s = 1.0 / det;
    double4 v = make_double4((a.w * bc.x + b.w * ca.x + d.w * ab.x) * s, (a.w * bc.y + b.w * ca.y + d.w * ab.y) * s,
                             (a.w * bc.z + b.w * ca.z + d.w * ab.z) * s, 0.0);
    v.w = dot_d(v, v);
    return v;
}

// The box planes 0..5 (+x, -x, +y, -y, +z, -z) and its 8 corners.  Corner
// (sx, sy, sz) is the triangle of planes (X, Y, Z), ordered X, Y, Z when an
// even number of them are "-" planes and X, Z, Y otherwise, so that every
// edge of the closed triangulation appears once in each direction.
__device__ __forceinline__ double4 box_plane(const VorGrid &g, double px, double py, double pz, int q)
{
    int a = q >> 1;
    double p = a == 0 ? px : (a == 1 ? py : pz);
    double4 pl = make_double4(0.0, 0.0, 0.0, (q & 1) ? p - g.box_lo[a] : g.box_hi[a] - p);
    (&pl.x)[a] = (q & 1) ? -1.0 : 1.0;
    return pl;
}
__device__ __forceinline__ uchar4 box_corner(int t)
{
    int sx = (t >> 2) & 1, sy = (t >> 1) & 1, sz = t & 1;
    uint8_t X = (uint8_t)sx, Y = (uint8_t)(2 + sy), Z = (uint8_t)(4 + sz);
    return ((sx + sy + sz) & 1) == 0 ? make_uchar4(X, Y, Z, 0) : make_uchar4(X, Z, Y, 0);
}
__device__ __forceinline__ double4 box_corner_pos(const VorGrid &g, double px, double py, double pz, int t)
{
    int sx = (t >> 2) & 1, sy = (t >> 1) & 1, sz = t & 1;
    double4 v = make_double4(sx ? g.box_lo[0] - px : g.box_hi[0] - px, sy ? g.box_lo[1] - py : g.box_hi[1] - py,
                             sz ? g.box_lo[2] - pz : g.box_hi[2] - pz, 0.0);
    v.w = dot_d(v, v);
    return v;
}

__device__ __forceinline__ int grid_coord(float x, float lo, float h, uint32_t g)
{
    int v = (int)floorf((x - lo) / h);
    return v < 0 ? 0 : (v >= (int)g ? (int)g - 1 : v);
}

// Grid cells of the row (dy, dz), relative to the site's cell (cx, ., .),
// that can hold sites at distances in [lo_g, hi_g) (grid units): up to two
// x ranges, [a0, a1] and [b0, b1] (empty when first > last).  A site in the
// cell at offset (dx, dy, dz) lies between (|dx|-1, |dy|-1, |dz|-1)+ and
// (|dx|+1, |dy|+1, |dz|+1) grid units away per axis; cells entirely inside
// lo_g were scanned by the earlier bands.  The margins of the callers cover
// the rounding of grid_coord at cell borders.
struct RowSpan {
    int a0, a1, b0, b1;
};
__device__ __forceinline__ bool band_row(int dy, int dz, double lo_g, double hi_g, int rr, int cx, int gx, RowSpan &s)
{
    double my = (double)max(abs(dy) - 1, 0), mz = (double)max(abs(dz) - 1, 0);
    double rem = hi_g * hi_g - my * my - mz * mz;
    if (rem <= 0.0)
        return false;
    int ro = min((int)floor(sqrt(rem)) + 1, rr);
    double py = (double)(abs(dy) + 1), pz = (double)(abs(dz) + 1);
    double rin = lo_g * lo_g - py * py - pz * pz;
    int si = rin > 0.0 ? (int)floor(sqrt(rin)) - 2 : -1;
    int lo = max(cx - ro, 0), hi = min(cx + ro, gx - 1);
    if (si < 0) {
        s.a0 = lo;
        s.a1 = hi;
        s.b0 = 1;
        s.b1 = 0;
    } else {
        s.a0 = lo;
        s.a1 = min(cx - si - 1, hi);
        s.b0 = max(cx + si + 1, lo);
        s.b1 = hi;
    }
    return true;
}

template <class Cap> struct WaveCell {
    double4 P[Cap::P];
    double4 V[Cap::T]; // w = |v|^2
    uint32_t nid[Cap::P];
    uchar4 T[Cap::T];
    alignas(8) uint16_t ed[Cap::E + 4]; // directed edges (u | v << 8) of the removed vertices
    uint16_t far[Cap::T];     // indices of the vertices beyond far2
    uint16_t slabfar[Cap::T]; // ... whose ball meets the current slab of grid cells
    uint16_t rowfar[Cap::T];  // ... and the current row
    uint32_t out[Cap::P];
    uint32_t run_off[64]; // candidates of one row piece: first candidate of lane l's grid cell
    uint32_t run_at[64];  // ... and where its sites start in the sorted order
    uint32_t used[8];
    uint32_t starts[Cap::P], ends[Cap::P]; // boundary edges per plane during a cut (0 otherwise)
    uint8_t remap[Cap::P];
    int np_shared;
};

__device__ __forceinline__ uint32_t lane_rank(uint64_t m)
{
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}
// Cross-lane move of a double by a DPP pattern within rows of 16 lanes.
template <int CTRL> __device__ __forceinline__ double dpp_d(double x)
{
    const uint64_t b = (uint64_t)__double_as_longlong(x);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, 0xf, 0xf, true);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, 0xf, 0xf, true);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double readlane_d(double x, int l)
{
    const uint64_t b = (uint64_t)__double_as_longlong(x);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
// Maximum over the wave (all lanes active): a butterfly within each row of
// 16 lanes (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_ror 4, row_ror 8),
// then the four row results.
__device__ __forceinline__ double wave_max_dpp(double x)
{
    x = fmax(x, dpp_d<0xb1>(x));
    x = fmax(x, dpp_d<0x4e>(x));
    x = fmax(x, dpp_d<0x124>(x));
    x = fmax(x, dpp_d<0x128>(x));
    return fmax(fmax(readlane_d(x, 0), readlane_d(x, 16)), fmax(readlane_d(x, 32), readlane_d(x, 48)));
}

// a value equal in every lane, moved to scalar registers
__device__ __forceinline__ double wave_uniform(double x)
{
    const uint64_t b = (uint64_t)__double_as_longlong(x);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Wave-uniform scalars of the cell (every lane holds the same values).
struct WaveState {
    int np, nt, nfar;
    int full;                // FULL_* bits of a capacity failure
    bool warm;               // guesses were cut in first (their sites come again)
    int gen;                 // effective cuts so far
    double R2, Rn2;          // squared radius of all vertices, of the near ones
    double bmin[3], bmax[3]; // bounding box of the near vertices (0 when none)
};

// R2, the near radius and bounding box and the far list, after a change.
template <class Cap> __device__ void wcell_radii(WaveCell<Cap> &c, WaveState &s, double far2, int lane)
{
    double r = 0.0, rn = 0.0;
    double mn[3] = {INFINITY, INFINITY, INFINITY}, mx[3] = {-INFINITY, -INFINITY, -INFINITY};
    int nf = 0;
    for (int t0 = 0; t0 < s.nt; t0 += 64) {
        const int t = t0 + lane;
        bool f = false;
        if (t < s.nt) {
            const double4 v = c.V[t];
            r = fmax(r, v.w);
            f = v.w > far2;
            if (!f) {
                rn = fmax(rn, v.w);
                mn[0] = fmin(mn[0], v.x);
                mn[1] = fmin(mn[1], v.y);
                mn[2] = fmin(mn[2], v.z);
                mx[0] = fmax(mx[0], v.x);
                mx[1] = fmax(mx[1], v.y);
                mx[2] = fmax(mx[2], v.z);
            }
        }
        uint64_t m = __ballot(f);
        if (f)
            c.far[nf + lane_rank(m)] = (uint16_t)t;
        nf += __popcll(m);
    }
    s.R2 = wave_uniform(wave_max_dpp(r));
    s.Rn2 = wave_uniform(wave_max_dpp(rn));
    const bool any_near = nf < s.nt;
    for (int a = 0; a < 3; ++a) {
        s.bmin[a] = any_near ? -wave_uniform(wave_max_dpp(-mn[a])) : 0.0;
        s.bmax[a] = any_near ? wave_uniform(wave_max_dpp(mx[a])) : 0.0;
    }
    s.nfar = nf;
    __syncthreads();
}

// Marks the planes that some vertex uses in c.used.
template <class Cap> __device__ void wcell_mark_used(WaveCell<Cap> &c, const WaveState &s, int lane)
{
    if (lane < 8)
        c.used[lane] = 0;
    __syncthreads();
    for (int t = lane; t < s.nt; t += 64) {
        uchar4 x = c.T[t];
        atomicOr(&c.used[x.x >> 5], 1u << (x.x & 31));
        atomicOr(&c.used[x.y >> 5], 1u << (x.y & 31));
        atomicOr(&c.used[x.z >> 5], 1u << (x.z & 31));
    }
    __syncthreads();
}

// Drop bisector planes that no vertex uses any more (the 6 box planes stay),
// renumbering the vertices' plane ids.  Called when the plane table is full.
template <class Cap> __device__ void wcell_compact_planes(WaveCell<Cap> &c, WaveState &s, int lane)
{
    wcell_mark_used(c, s, lane);
    if (lane == 0) {
        int m = 6;
        for (int q = 0; q < 6; ++q)
            c.remap[q] = (uint8_t)q;
        for (int q = 6; q < s.np; ++q) {
            if (c.used[q >> 5] & (1u << (q & 31))) {
                c.P[m] = c.P[q];
                c.nid[m] = c.nid[q];
                c.remap[q] = (uint8_t)m++;
            }
        }
        c.np_shared = m;
    }
    __syncthreads();
    for (int t = lane; t < s.nt; t += 64) {
        uchar4 x = c.T[t];
        c.T[t] = make_uchar4(c.remap[x.x], c.remap[x.y], c.remap[x.z], 0);
    }
    s.np = c.np_shared;
    __syncthreads();
}

// Cut by n.x <= w, spread over the wave.  Returns a wave-uniform status
// (VOR_OK also when the plane misses the cell).
template <class Cap, bool WARM>
__device__ int wcell_cut(WaveCell<Cap> &c, WaveState &s, double4 pl, uint32_t site, double far2, int lane)
{
    if (WARM && s.warm) {
        // The band scan offers a guessed site again.  Its plane is already a
        // face; a vertex on it may round to "outside", and cutting the same
        // plane again would make a vertex of parallel planes.
        bool dup = false;
        for (int q = 6 + lane; q < s.np; q += 64)
            dup = dup || c.nid[q] == site;
        if (__ballot(dup))
            return VOR_OK;
    }
    if (s.np >= Cap::P) {
        wcell_compact_planes(c, s, lane);
        if (s.np >= Cap::P) {
            s.full |= FULL_PLANES;
            return VOR_FULL;
        }
    }
    // classify; gather the edges of the removed vertices
    uint32_t outmask = 0; // bit b: vertex 64 b + lane is removed
    int removed = 0;
    for (int t0 = 0, b = 0; t0 < s.nt; t0 += 64, ++b) {
        const int t = t0 + lane;
        bool out = false;
        uchar4 x = make_uchar4(0, 0, 0, 0);
        if (t < s.nt) {
            out = dot_d(pl, c.V[t]) > pl.w;
            x = c.T[t];
        }
        uint64_t m = __ballot(out);
        const int cnt = __popcll(m);
        if (3 * (removed + cnt) > Cap::E) {
            s.full |= FULL_EDGES;
            return VOR_FULL;
        }
        if (out) {
            const int e = 3 * (removed + (int)lane_rank(m));
            c.ed[e] = (uint16_t)(x.x | (x.y << 8));
            c.ed[e + 1] = (uint16_t)(x.y | (x.z << 8));
            c.ed[e + 2] = (uint16_t)(x.z | (x.x << 8));
            outmask |= 1u << b;
        }
        removed += cnt;
    }
    if (removed == 0)
        return VOR_OK;
    if (removed == s.nt)
        return VOR_DEGENERATE; // the site's own half-space always keeps the site
    const int ne = 3 * removed;
    const int q = s.np++;
    if (lane == 0) {
        c.P[q] = pl;
        c.nid[q] = site;
    }
    if (lane < 4)
        c.ed[ne + lane] = 0xffff; // plane ids are below 255
    // compact the kept vertices (a chunk is read before it is written; the
    // writes land below the next chunk)
    int k = 0;
    for (int t0 = 0, b = 0; t0 < s.nt; t0 += 64, ++b) {
        const int t = t0 + lane;
        const bool keep = t < s.nt && !((outmask >> b) & 1u);
        uchar4 x = make_uchar4(0, 0, 0, 0);
        double4 v = make_double4(0.0, 0.0, 0.0, 0.0);
        if (keep) {
            x = c.T[t];
            v = c.V[t];
        }
        uint64_t m = __ballot(keep);
        __syncthreads();
        if (keep) {
            const int d = k + (int)lane_rank(m);
            c.T[d] = x;
            c.V[d] = v;
        }
        k += __popcll(m);
    }
    __syncthreads(); // edges, plane q and kept vertices visible to all lanes
    // boundary edges (u, v): their reverse belongs to a kept vertex; the new
    // vertex (u, v, q) keeps the orientation.  A cut of a convex cell removes
    // a disc, so the boundary is one cycle: every plane on it starts exactly
    // one edge and ends exactly one.
    int nb = 0;
    for (int e0 = 0; e0 < ne; e0 += 64) {
        const int e = e0 + lane;
        bool bnd = false;
        uint16_t ev = 0;
        if (e < ne) {
            ev = c.ed[e];
            const uint64_t rev = (uint64_t)((ev >> 8) | ((ev & 0xff) << 8)) * 0x0001000100010001ull;
            const uint64_t *e4 = reinterpret_cast<const uint64_t *>(c.ed);
            uint64_t hit = 0;
            for (int f = 0; f < ne; f += 4) {
                const uint64_t x = e4[f >> 2] ^ rev; // a zero field: the reverse edge
                hit |= (x - 0x0001000100010001ull) & ~x & 0x8000800080008000ull;
            }
            bnd = hit == 0;
        }
        uint64_t m = __ballot(bnd);
        const int cnt = __popcll(m);
        if (k + nb + cnt > Cap::T) {
            s.full |= FULL_VERTICES;
            return VOR_FULL;
        }
        if (bnd)
            c.T[k + nb + (int)lane_rank(m)] = make_uchar4((uint8_t)(ev & 0xff), (uint8_t)(ev >> 8), (uint8_t)q, 0);
        nb += cnt;
    }
    if (nb < 3)
        return VOR_DEGENERATE;
    __syncthreads();
    for (int a = k + lane; a < k + nb; a += 64) {
        const uchar4 x = c.T[a];
        atomicAdd(&c.starts[x.x], 1u);
        atomicAdd(&c.ends[x.y], 1u);
    }
    __syncthreads();
    bool bad = false;
    for (int a = k + lane; a < k + nb; a += 64) {
        const uint8_t u = c.T[a].x;
        bad = bad || c.starts[u] != 1u || c.ends[u] != 1u;
    }
    __syncthreads();
    for (int a = k + lane; a < k + nb; a += 64) {
        const uchar4 x = c.T[a];
        c.starts[x.x] = 0u;
        c.ends[x.y] = 0u;
    }
    if (__ballot(bad))
        return VOR_DEGENERATE;
    for (int a = k + lane; a < k + nb; a += 64) {
        const uchar4 x = c.T[a];
        const double4 v = plane_vertex(c.P[x.x], c.P[x.y], c.P[x.z]);
        bad = bad || !(v.w < 1e300); // a vertex of (nearly) parallel planes
        c.V[a] = v;
    }
    if (__ballot(bad))
        return VOR_DEGENERATE;
    s.nt = k + nb;
    ++s.gen;
    __syncthreads();
    wcell_radii(c, s, far2, lane);
    return VOR_OK;
}

// max of x.v over x in [l, h] and v in [bmin, bmax], one axis
__device__ __forceinline__ double axis_support(double l, double h, double bmin, double bmax)
{
    return fmax(fmax(l * bmin, l * bmax), fmax(h * bmin, h * bmax));
}

// A box of space (local coordinates, widened by the grid rounding margin):
// the distances of its points from the site.
struct VorBox {
    double lo[3], hi[3];
    double mind2, maxd2;
    __device__ void finish()
    {
        mind2 = maxd2 = 0.0;
        for (int a = 0; a < 3; ++a) {
            const double near = lo[a] > 0.0 ? lo[a] : (hi[a] < 0.0 ? -hi[a] : 0.0);
            const double farc = fmax(-lo[a], hi[a]);
            mind2 += near * near;
            maxd2 += farc * farc;
        }
    }
    // Could a site of the band [lo2, hi2) in the box cut the cell at all?
    __device__ bool in_reach(const WaveState &s, double lo2, double hi2) const
    {
        return mind2 < hi2 && maxd2 >= lo2 && mind2 < 4.0 * s.R2;
    }
    // Could a site in the box cut a near vertex?  A cut of v needs
    // x.v > |x|^2 / 2; max x.v is bounded through the bounding box of the
    // near vertices (slack for the rounding of the bound).
    __device__ bool near_may_cut(const WaveState &s) const
    {
        if (s.nfar >= s.nt)
            return false;
        const double sb = axis_support(lo[0], hi[0], s.bmin[0], s.bmax[0]) +
                          axis_support(lo[1], hi[1], s.bmin[1], s.bmax[1]) +
                          axis_support(lo[2], hi[2], s.bmin[2], s.bmax[2]);
        return sb >= 0.5 * mind2 * (1.0 - 1e-9);
    }
    // Could a site in the box cut vertex v: does the box meet the ball
    // B(v, |v|) (the sites closer to v than the cell's own site)?
    __device__ bool meets_ball(double4 v) const
    {
        const double ax = fmax(fmax(lo[0] - v.x, v.x - hi[0]), 0.0);
        const double ay = fmax(fmax(lo[1] - v.y, v.y - hi[1]), 0.0);
        const double az = fmax(fmax(lo[2] - v.z, v.z - hi[2]), 0.0);
        return ax * ax + ay * ay + az * az < v.w * (1.0 + 1e-9);
    }
};

// The far vertices of src[0..nsrc) whose ball meets the box go to dst
// (spread over the lanes); returns their number.  The caller synchronises
// before (dst may still be read) and after.
template <class Cap>
__device__ int collect_far(const WaveCell<Cap> &c, const uint16_t *src, int nsrc, uint16_t *dst, const VorBox &b,
                           int lane)
{
    int n = 0;
    for (int f0 = 0; f0 < nsrc; f0 += 64) {
        const int f = f0 + lane;
        bool m = false;
        uint16_t id = 0;
        if (f < nsrc) {
            id = src[f];
            m = b.meets_ball(c.V[id]);
        }
        const uint64_t bm = __ballot(m);
        if (m)
            dst[n + (int)lane_rank(bm)] = id;
        n += __popcll(bm);
    }
    return n;
}

// Does the plane of d (d.x <= |d|^2 / 2) cut the cell?  Far vertices are
// those of the list (the ones the site's row can reach).
template <class Cap>
__device__ __forceinline__ bool wcell_hits(const WaveCell<Cap> &c, const WaveState &s, const uint16_t *far,
                                           int nfar, double dx, double dy, double dz, double d2)
{
    const double w = 0.5 * d2;
    bool hit = false;
    for (int f = 0; f < nfar; ++f) {
        const double4 v = c.V[far[f]];
        hit |= dx * v.x + dy * v.y + dz * v.z > w;
    }
    if (!hit && d2 < 4.0 * s.Rn2) {
        const double sb = fmax(dx * s.bmin[0], dx * s.bmax[0]) + fmax(dy * s.bmin[1], dy * s.bmax[1]) +
                          fmax(dz * s.bmin[2], dz * s.bmax[2]);
        if (sb * (1.0 + 1e-9) > w) {
#pragma unroll 4
            for (int t = 0; t < s.nt; ++t) {
                const double4 v = c.V[t];
                hit |= dx * v.x + dy * v.y + dz * v.z > w;
            }
        }
    }
    return hit;
}

// Voronoi cell of site i; its m neighbours go to c.out[0..m) (unordered).
// Cuts of the candidates of `m` (bit l: lane l's plane, site j, offset d,
// |d|^2 = d2), nearest first: the nearer planes make many farther ones miss.
template <class Cap, bool WARM>
__device__ __forceinline__ int cut_nearest_first(WaveCell<Cap> &c, WaveState &s, uint64_t m, uint32_t j, double ddx,
                                                 double ddy, double ddz, double d2, double far2, int lane)
{
    int status = VOR_OK;
    while (m && status == VOR_OK) {
        int l = __ffsll((unsigned long long)m) - 1;
        if (m & (m - 1)) {
            const bool rem = (m >> lane) & 1u;
            const double dmin = -wave_max_dpp(rem ? -d2 : -INFINITY);
            l = __ffsll((unsigned long long)__ballot(rem && d2 == dmin)) - 1;
        }
        m &= ~(1ull << l);
        const double4 pl = make_double4(__shfl(ddx, l), __shfl(ddy, l), __shfl(ddz, l), 0.5 * __shfl(d2, l));
        status = wcell_cut<Cap, WARM>(c, s, pl, (uint32_t)__shfl((int)j, l), far2, lane);
    }
    return status;
}

// Warm start: the cell is first cut by the guessed neighbours of site i
// (gadj[gofs[i], gofs[i+1]), e.g. the adjacency before the sites moved),
// nearest first.  Every bisector plane is a valid constraint of the cell, and the
// band scan that follows still tests every site that could cut it, so the
// result is the cell without guesses; with good guesses the scan meets a
// cell that is already final (small R, few candidates that still cut).
template <class Cap>
__device__ int wave_guess_cuts(WaveCell<Cap> &c, WaveState &s, uint32_t i, const float *__restrict__ points,
                               uint32_t n, const uint32_t *__restrict__ gofs, const uint32_t *__restrict__ gadj,
                               double px, double py, double pz, double far2, int lane)
{
    const uint32_t gb = gofs[i], ge = gofs[i + 1];
    int status = VOR_OK;
    for (uint32_t kb = gb; kb < ge && status == VOR_OK; kb += 64) {
        const uint32_t k = kb + (uint32_t)lane;
        bool cand = false;
        uint32_t j = 0;
        double ddx = 0.0, ddy = 0.0, ddz = 0.0, d2 = 0.0;
        if (k < ge) {
            j = gadj[k];
            if (j < n && j != i) {
                ddx = (double)points[3 * j] - px;
                ddy = (double)points[3 * j + 1] - py;
                ddz = (double)points[3 * j + 2] - pz;
                d2 = ddx * ddx + ddy * ddy + ddz * ddz;
                cand = d2 > 0.0 && wcell_hits(c, s, c.far, s.nfar, ddx, ddy, ddz, d2);
            }
        }
        status = cut_nearest_first<Cap, true>(c, s, __ballot(cand), j, ddx, ddy, ddz, d2, far2, lane);
    }
    return status;
}

template <class Cap, bool WARM>
__device__ int wave_voronoi_cell(WaveCell<Cap> &c, uint32_t i, const float *__restrict__ points, const VorGrid &g,
                                 const uint32_t *__restrict__ cell_start, const uint32_t *__restrict__ sorted,
                                 uint32_t n, const uint32_t *__restrict__ gofs, const uint32_t *__restrict__ gadj,
                                 int lane, int *m_out, int *full_out)
{
    const float pxf = points[3 * i], pyf = points[3 * i + 1], pzf = points[3 * i + 2];
    const double px = pxf, py = pyf, pz = pzf;
    WaveState s;
    if (lane < 6) {
        c.P[lane] = box_plane(g, px, py, pz, lane);
        c.nid[lane] = VOR_NONE;
    }
    if (lane < 8) {
        c.T[lane] = box_corner(lane);
        c.V[lane] = box_corner_pos(g, px, py, pz, lane);
    }
    for (int q = lane; q < Cap::P; q += 64)
        c.starts[q] = c.ends[q] = 0u;
    s.np = 6;
    s.nt = 8;
    s.gen = 0;
    s.full = 0;
    s.warm = gofs != nullptr;
    __syncthreads();
    wcell_radii(c, s, g.far2, lane);
    const int cx = grid_coord(pxf, g.lo[0], g.h, g.g[0]);
    const int cy = grid_coord(pyf, g.lo[1], g.h, g.g[1]);
    const int cz = grid_coord(pzf, g.lo[2], g.h, g.g[2]);
    const int gmax = (int)max(g.g[0], max(g.g[1], g.g[2]));
    const double h = (double)g.h;
    const double eps = 1e-3 * h; // grid rounding margin
    const double diag2 = (double)(g.g[0] * g.g[0] + g.g[1] * g.g[1] + g.g[2] * g.g[2]) * h * h;
    // local box of the grid cells [x0, x1] x [y0, y1] x [z0, z1]
    auto cells_box = [&](int x0, int x1, int y0, int y1, int z0, int z1) {
        VorBox b;
        b.lo[0] = (double)g.lo[0] + x0 * h - px - eps;
        b.hi[0] = (double)g.lo[0] + (x1 + 1) * h - px + eps;
        b.lo[1] = (double)g.lo[1] + y0 * h - py - eps;
        b.hi[1] = (double)g.lo[1] + (y1 + 1) * h - py + eps;
        b.lo[2] = (double)g.lo[2] + z0 * h - pz - eps;
        b.hi[2] = (double)g.lo[2] + (z1 + 1) * h - pz + eps;
        b.finish();
        return b;
    };
    int status = VOR_OK;
    if constexpr (WARM) {
        if (gofs)
            status = wave_guess_cuts(c, s, i, points, n, gofs, gadj, px, py, pz, g.far2, lane);
    }
    double lo2 = 0.0;
    double rho0 = 0.125 * h;
    if (WARM && gofs && status == VOR_OK) {
        // The guesses usually leave the cell near its final shape: one shell
        // of radius 2R (R = farthest vertex) then finishes the scan, where
        // doubling from h/8 would visit the same rows several times.  Poor
        // guesses (a large R) keep the doubling schedule.
        const double r2 = 2.0 * sqrt(s.R2) * (1.0 + 1e-6);
        if (r2 <= 4.0 * h)
            rho0 = fmax(rho0, r2);
    }
    for (double rho = rho0; status == VOR_OK; rho *= 2.0) {
        const double hi2 = rho * rho;
        const double hig = rho / h + 1e-3, log_ = fmax(sqrt(lo2) / h - 1e-3, 0.0);
        const int rr = min((int)ceil(hig), gmax);
        const int gx0 = max(cx - rr, 0), gx1 = min(cx + rr, (int)g.g[0] - 1);
        const int gy0 = max(cy - rr, 0), gy1 = min(cy + rr, (int)g.g[1] - 1);
        // rows nearest first (0, -1, +1, -2, +2, ...): their sites cut the
        // cell early, so fewer planes of farther sites cut it only to be
        // superseded (the cell does not depend on the order)
        for (int zi = 0; zi <= 2 * rr && status == VOR_OK; ++zi) {
            const int dz = (zi & 1) ? -((zi + 1) >> 1) : (zi >> 1);
            const int z = cz + dz;
            if (z < 0 || z >= (int)g.g[2])
                continue;
            // the slab of the band at this z: its far vertices
            const VorBox slab = cells_box(gx0, gx1, gy0, gy1, z, z);
            if (!slab.in_reach(s, lo2, hi2))
                continue;
            int nsf = 0, nrf = 0;
            auto refresh_slab = [&]() {
                __syncthreads();
                nsf = collect_far(c, c.far, s.nfar, c.slabfar, slab, lane);
                __syncthreads();
            };
            refresh_slab();
            if (nsf == 0 && !slab.near_may_cut(s))
                continue;
            int lgen = s.gen; // cut generation the lists belong to
            for (int yi = 0; yi <= 2 * rr && status == VOR_OK; ++yi) {
                const int dy = (yi & 1) ? -((yi + 1) >> 1) : (yi >> 1);
                const int y = cy + dy;
                RowSpan sp;
                if (y < 0 || y >= (int)g.g[1] || !band_row(dy, dz, log_, hig, rr, cx, (int)g.g[0], sp))
                    continue;
                const int rx0 = sp.a0 <= sp.a1 ? sp.a0 : sp.b0, rx1 = sp.b0 <= sp.b1 ? sp.b1 : sp.a1;
                if (rx0 > rx1)
                    continue;
                const VorBox rowb = cells_box(rx0, rx1, y, y, z, z);
                if (!rowb.in_reach(s, lo2, hi2))
                    continue;
                // after a cut the vertex indices of the lists are stale
                auto refresh_row = [&]() {
                    if (lgen != s.gen) {
                        refresh_slab();
                        lgen = s.gen;
                    }
                    nrf = collect_far(c, c.slabfar, nsf, c.rowfar, rowb, lane);
                    __syncthreads();
                };
                refresh_row();
                if (nrf == 0 && !rowb.near_may_cut(s))
                    continue;
                const uint32_t row = ((uint32_t)z * g.g[1] + (uint32_t)y) * g.g[0];
                for (int part = 0; part < 2 && status == VOR_OK; ++part) {
                    const int x0 = part ? sp.b0 : sp.a0, x1 = part ? sp.b1 : sp.a1;
                    for (int xb = x0; xb <= x1 && status == VOR_OK; xb += 64) {
                        if (lgen != s.gen)
                            refresh_row();
                        // lane = grid cell of the row piece; surviving cells'
                        // sites are packed into consecutive candidates
                        const int x = xb + lane;
                        uint32_t at = 0, cnt = 0;
                        if (x <= x1) {
                            const VorBox cb = cells_box(x, x, y, y, z, z);
                            bool may = cb.in_reach(s, lo2, hi2) && cb.near_may_cut(s);
                            for (int f = 0; f < nrf && !may; ++f)
                                may = cb.meets_ball(c.V[c.rowfar[f]]);
                            if (may && cb.in_reach(s, lo2, hi2)) {
                                at = cell_start[row + x];
                                cnt = cell_start[row + x + 1] - at;
                            }
                        }
                        uint32_t incl = cnt;
                        for (int o = 1; o < 64; o <<= 1) {
                            const uint32_t v = __shfl_up(incl, o);
                            if (lane >= o)
                                incl += v;
                        }
                        const uint32_t total = __shfl(incl, 63);
                        if (total == 0)
                            continue;
                        c.run_off[lane] = incl - cnt;
                        c.run_at[lane] = at;
                        __syncthreads();
                        for (uint32_t kb = 0; kb < total && status == VOR_OK; kb += 64) {
                            if (lgen != s.gen)
                                refresh_row();
                            const uint32_t kk = kb + (uint32_t)lane;
                            bool cand = false;
                            uint32_t j = 0;
                            double ddx = 0.0, ddy = 0.0, ddz = 0.0, d2 = 0.0;
                            if (kk < total) {
                                int L = 0; // last lane whose run starts at or before kk
                                for (int step = 32; step > 0; step >>= 1)
                                    if (c.run_off[L + step] <= kk)
                                        L += step;
                                j = sorted[c.run_at[L] + (kk - c.run_off[L])];
                                ddx = (double)points[3 * j] - px;
                                ddy = (double)points[3 * j + 1] - py;
                                ddz = (double)points[3 * j + 2] - pz;
                                d2 = ddx * ddx + ddy * ddy + ddz * ddz;
                                cand = j != i && d2 >= lo2 && d2 < hi2 && d2 < 4.0 * s.R2 &&
                                       wcell_hits(c, s, c.rowfar, nrf, ddx, ddy, ddz, d2);
                            }
                            status = cut_nearest_first<Cap, WARM>(c, s, __ballot(cand), j, ddx, ddy, ddz, d2, g.far2,
                                                       lane);
                        }
                        __syncthreads(); // run_off / run_at are rewritten by the next piece
                    }
                }
            }
        }
        if (status != VOR_OK || 4.0 * s.R2 <= hi2 || hi2 > diag2)
            break;
        lo2 = hi2;
    }
    int m = 0;
    if (status == VOR_OK) {
        wcell_mark_used(c, s, lane);
        for (int q0 = 6; q0 < s.np; q0 += 64) {
            const int q = q0 + lane;
            const bool u = q < s.np && ((c.used[q >> 5] >> (q & 31)) & 1u);
            uint64_t mm = __ballot(u);
            if (u)
                c.out[m + (int)lane_rank(mm)] = c.nid[q];
            m += __popcll(mm);
        }
        __syncthreads();
    }
    *m_out = status == VOR_OK ? m : 0;
    *full_out = s.full;
    return status;
}

// One wave per cell, cells taken in order from a work counter.  First pass
// (LARGE false): every site, in the layer order; cells that overflow the small
// tables are queued in retry[].  Second pass (LARGE true): the queued cells.
// A list longer than LIST_K goes to a slot of big_lists (big_slot[i]),
// shorter lists to the cell's slot of lists.
template <class Cap, bool LARGE, bool WARM>
__global__ __launch_bounds__(VOR_BLOCK) __attribute__((amdgpu_waves_per_eu(LARGE ? 1 : 3))) void voronoi_cells_kernel(
    const float *__restrict__ points, VorGrid g, const uint32_t *__restrict__ cell_start,
    const uint32_t *__restrict__ sorted, const uint32_t *__restrict__ cells, uint32_t ncells,
    uint32_t *__restrict__ lists, uint32_t *__restrict__ big_lists, uint32_t big_cap, uint32_t *__restrict__ big_slot,
    uint32_t *__restrict__ counts, uint32_t *__restrict__ retry, uint32_t *fails, uint32_t n,
    const uint32_t *__restrict__ gofs, const uint32_t *__restrict__ gadj, uint32_t gcount)
{
    __shared__ WaveCell<Cap> c;
    __shared__ uint32_t pick;
    const int lane = (int)threadIdx.x;
    uint32_t *next = fails + (LARGE ? F_NEXT1 : F_NEXT0);
    for (;;) {
        if (lane == 0)
            pick = atomicAdd(next, 1u);
        __syncthreads();
        const uint32_t r = pick;
        __syncthreads();
        if (r >= ncells)
            break;
        const uint32_t i = cells[r];
        int m;
        // Guesses seed the first pass only, and only cells with at most 64 of
        // them (one nearest-first group): a longer list cut group by group can
        // hold more vertices on the way than the cold band order, and the
        // retry with the large tables runs cold, so guesses never cause a
        // capacity failure.  A range that runs backwards or past the gcount
        // guesses is not read (the cell builds cold).
        bool warm = false;
        if (WARM && !LARGE) {
            const uint32_t gb = gofs[i], ge = gofs[i + 1];
            warm = gb <= ge && ge <= gcount && ge - gb <= 64u;
        }
        int full = 0;
        int status = wave_voronoi_cell<Cap, WARM>(c, i, points, g, cell_start, sorted, n, warm ? gofs : nullptr,
                                                  gadj, lane, &m, &full);
        uint32_t *dst = lists + (size_t)i * LIST_K;
        if (status == VOR_OK && m > LIST_K) {
            if (lane == 0)
                pick = atomicAdd(fails + F_BIG, 1u);
            __syncthreads();
            const uint32_t slot = pick;
            __syncthreads();
            if (slot < big_cap) {
                dst = big_lists + (size_t)slot * BIG_K;
                if (lane == 0)
                    big_slot[i] = slot;
            } else {
                status = VOR_FULL;
                full |= FULL_LISTS;
            }
        }
        if (status == VOR_OK) {
            // ascending by rank (the ids are distinct)
            for (int a = lane; a < m; a += 64) {
                const uint32_t v = c.out[a];
                int rank = 0;
                for (int b = 0; b < m; ++b)
                    rank += c.out[b] < v;
                dst[rank] = v;
            }
        } else {
            m = 0;
            if (lane == 0) {
                if (!LARGE && status == VOR_FULL)
                    retry[atomicAdd(fails + F_RETRY, 1u)] = i; // at most n entries
                else {
                    atomicAdd(fails + (status == VOR_FULL ? F_FULL : F_DEGENERATE), 1u);
                    atomicMin(fails + F_FIRST_BAD, i);
                    atomicOr(fails + F_REASON, (uint32_t)full);
                }
            }
        }
        if (lane == 0)
            counts[i] = (uint32_t)m;
        __syncthreads();
    }
}

__global__ void voronoi_grid_keys_kernel(const float *__restrict__ points, uint32_t n, VorGrid g,
                                         uint32_t *__restrict__ keys, uint32_t *__restrict__ vals,
                                         uint32_t *__restrict__ cell_count)
{
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n)
        return;
    int x = grid_coord(points[3 * i], g.lo[0], g.h, g.g[0]);
    int y = grid_coord(points[3 * i + 1], g.lo[1], g.h, g.g[1]);
    int z = grid_coord(points[3 * i + 2], g.lo[2], g.h, g.g[2]);
    uint32_t cell = ((uint32_t)z * g.g[1] + (uint32_t)y) * g.g[0] + (uint32_t)x;
    keys[i] = cell;
    vals[i] = i;
    atomicAdd(cell_count + cell, 1u);
}

// Work order of the cells: by grid layer (distance of the grid cell from the
// grid's boundary, outermost first: the long cells of convex-hull sites start
// early instead of trailing the pass), grid order within a layer.
__global__ void voronoi_layer_kernel(uint32_t *__restrict__ keys, const uint32_t *__restrict__ vals, uint32_t n,
                                     VorGrid g, uint32_t *__restrict__ order)
{
    uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n)
        return;
    const uint32_t cell = keys[t];
    const int x = (int)(cell % g.g[0]), y = (int)((cell / g.g[0]) % g.g[1]), z = (int)(cell / (g.g[0] * g.g[1]));
    const int layer = min(min(min(x, (int)g.g[0] - 1 - x), min(y, (int)g.g[1] - 1 - y)), min(z, (int)g.g[2] - 1 - z));
    keys[t] = (uint32_t)min(layer, 255);
    order[t] = vals[t];
}

__global__ void voronoi_copy_kernel(uint32_t n, const uint32_t *__restrict__ offsets,
                                    const uint32_t *__restrict__ lists, const uint32_t *__restrict__ big_lists,
                                    const uint32_t *__restrict__ big_slot, uint32_t *__restrict__ adjacency)
{
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n)
        return;
    uint32_t b = offsets[i], m = offsets[i + 1] - b;
    uint32_t slot = big_slot[i];
    const uint32_t *src = slot == VOR_NONE ? lists + (size_t)i * LIST_K : big_lists + (size_t)slot * BIG_K;
    for (uint32_t k = 0; k < m; ++k)
        adjacency[b + k] = src[k];
}

__global__ void fill_u32_kernel(uint32_t *p, size_t n, uint32_t v)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        p[i] = v;
}

// workspace layout (u32 words)
struct VorWs {
    uint32_t *lists, *counts, *keys, *vals, *cell_start, *sort_ws, *scan_ws, *fails, *bbox_ws, *retry, *big_lists,
        *big_slot, *order;
    float *bbox;
};

static uint32_t grid_cells_for(uint32_t n) { return n < 8 ? 8 : n; }
// cells with more than LIST_K neighbours
static uint32_t big_cap_for(uint32_t n) { return std::max<uint32_t>(256, n / 64); }

static size_t ws_words(uint32_t n, VorWs *w, uint32_t *base)
{
    size_t cells = grid_cells_for(n) + 2 * 512 * 512; // slack for non-cubic boxes
    size_t off = 0;
    uint32_t *dummy;
    auto take = [&](uint32_t **p, size_t words) {
        *(w ? p : &dummy) = base + off;
        off += (words + 63) & ~(size_t)63;
    };
    VorWs local{};
    VorWs &x = w ? *w : local;
    take(&x.lists, (size_t)n * LIST_K);
    take(&x.counts, (size_t)n + 1);
    take(&x.keys, n);
    take(&x.vals, n);
    take(&x.cell_start, cells + 1);
    take(&x.sort_ws, radix_sort_workspace_words(n));
    take(&x.scan_ws, scan_workspace_words((uint32_t)std::max<size_t>(cells + 1, (size_t)n + 1)));
    take(&x.fails, F_WORDS);
    take(&x.bbox_ws, 6);
    uint32_t *bb;
    take(&bb, 6);
    x.bbox = reinterpret_cast<float *>(bb);
    take(&x.retry, n);
    take(&x.big_lists, (size_t)big_cap_for(n) * BIG_K);
    take(&x.big_slot, n);
    take(&x.order, n);
    return off;
}

// enough waves to fill the chip (the LDS of a cell bounds them per CU)
static uint32_t wave_blocks(uint32_t ncells) { return std::min<uint32_t>(ncells, 256u * 16u); }

} // namespace vt

using namespace vt;

extern "C" size_t vt_voronoi_workspace_size(uint32_t num_points)
{
    return ws_words(num_points, nullptr, nullptr) * sizeof(uint32_t);
}

extern "C" int vt_voronoi_build(const float *points, uint32_t num_points, uint32_t *offsets,
                                uint32_t *num_adjacency, void *workspace, vt_stream_t stream)
{
    return vt_voronoi_build_warm(points, num_points, nullptr, nullptr, 0, offsets, num_adjacency, workspace, stream);
}

extern "C" int vt_voronoi_build_warm(const float *points, uint32_t num_points, const uint32_t *guess_offsets,
                                     const uint32_t *guess_adjacency, uint32_t num_guesses, uint32_t *offsets,
                                     uint32_t *num_adjacency,
                                     void *workspace, vt_stream_t stream)
{
    clear_error();
    VT_REQUIRE(points && offsets && num_adjacency && workspace, "null pointer argument");
    VT_REQUIRE(!guess_offsets == !guess_adjacency, "guess offsets and adjacency are given together or not at all");
    VT_REQUIRE(num_points >= 2, "at least 2 sites are needed, got %u", num_points);
    VT_REQUIRE(num_points <= (1u << 26), "too many sites (%u)", num_points);
    hipStream_t s = as_stream(stream);
    VorWs w{};
    ws_words(num_points, &w, reinterpret_cast<uint32_t *>(workspace));
    uint32_t n = num_points;
    // bounding box -> grid of about one site per cell
    int rc = bbox3(points, n, w.bbox, w.bbox_ws, s);
    if (rc)
        return rc;
    float bb[6];
    VT_HIP_CHECK(hipMemcpyAsync(bb, w.bbox, sizeof(bb), hipMemcpyDeviceToHost, s));
    VT_HIP_CHECK(hipStreamSynchronize(s));
    VorGrid g{};
    double ext[3], vol = 1.0, maxext = 0.0;
    for (int a = 0; a < 3; ++a) {
        ext[a] = std::max((double)bb[3 + a] - (double)bb[a], 1e-6);
        vol *= ext[a];
        maxext = std::max(maxext, ext[a]);
    }
    double h = std::cbrt(vol / (double)n);
    uint64_t cells = 1;
    for (int a = 0; a < 3; ++a) {
        g.g[a] = (uint32_t)std::max(1.0, std::min(512.0, std::ceil(ext[a] / h)));
        cells *= g.g[a];
    }
    for (int a = 0; a < 3; ++a) {
        g.lo[a] = bb[a];
        g.box_lo[a] = (double)bb[a] - 1e6 * maxext;
        g.box_hi[a] = (double)bb[3 + a] + 1e6 * maxext;
    }
    g.h = (float)std::max({ext[0] / g.g[0], ext[1] / g.g[1], ext[2] / g.g[2]}) * 1.0000001f;
    // vertices farther than 4 grid cells (box vertices, the long cells of
    // convex-hull sites) are tested one by one rather than through the
    // bounding box of the others
    g.far2 = 16.0 * (double)g.h * (double)g.h;
    VT_REQUIRE(cells <= (uint64_t)grid_cells_for(n) + 2ull * 512 * 512, "grid too large");
    uint32_t nc = (uint32_t)cells;
    // bucket the sites by grid cell: counts -> starts; stable sort of (cell, site)
    fill_u32_kernel<<<(nc + 1 + 255) / 256, 256, 0, s>>>(w.cell_start, (size_t)nc + 1, 0u);
    fill_u32_kernel<<<1, 64, 0, s>>>(w.fails, F_WORDS, 0u);
    fill_u32_kernel<<<1, 64, 0, s>>>(w.fails + F_FIRST_BAD, 1, VOR_NONE);
    fill_u32_kernel<<<(n + 255) / 256, 256, 0, s>>>(w.big_slot, n, VOR_NONE);
    voronoi_grid_keys_kernel<<<(n + 255) / 256, 256, 0, s>>>(points, n, g, w.keys, w.vals, w.cell_start);
    VT_LAUNCH_CHECK("voronoi_grid_keys_kernel");
    rc = exclusive_scan_u32(w.cell_start, w.cell_start, nc + 1, w.scan_ws, s);
    if (rc)
        return rc;
    int bits = 1;
    while (bits < 32 && (1ull << bits) < nc)
        ++bits;
    rc = radix_sort_pairs(w.keys, w.vals, n, bits, w.sort_ws, s);
    if (rc)
        return rc;
    voronoi_layer_kernel<<<(n + 255) / 256, 256, 0, s>>>(w.keys, w.vals, n, g, w.order);
    VT_LAUNCH_CHECK("voronoi_layer_kernel");
    rc = radix_sort_pairs(w.keys, w.order, n, 8, w.sort_ws, s);
    if (rc)
        return rc;
    const uint32_t bcap = big_cap_for(n);
    // cold builds run an instantiation without any of the warm-start code
    if (guess_offsets)
        voronoi_cells_kernel<VorSmall, false, true><<<wave_blocks(n), VOR_BLOCK, 0, s>>>(
            points, g, w.cell_start, w.vals, w.order, n, w.lists, w.big_lists, bcap, w.big_slot, w.counts, w.retry,
            w.fails, n, guess_offsets, guess_adjacency, num_guesses);
    else
        voronoi_cells_kernel<VorSmall, false, false><<<wave_blocks(n), VOR_BLOCK, 0, s>>>(
            points, g, w.cell_start, w.vals, w.order, n, w.lists, w.big_lists, bcap, w.big_slot, w.counts, w.retry,
            w.fails, n, nullptr, nullptr, 0u);
    VT_LAUNCH_CHECK("voronoi_cells_kernel (small)");
    uint32_t f[F_WORDS];
    VT_HIP_CHECK(hipMemcpyAsync(f, w.fails, sizeof(f), hipMemcpyDeviceToHost, s));
    VT_HIP_CHECK(hipStreamSynchronize(s));
    if (f[F_RETRY]) {
        // the retry pass runs cold (guesses never cause a capacity failure)
        voronoi_cells_kernel<VorLarge, true, false><<<wave_blocks(f[F_RETRY]), VOR_BLOCK, 0, s>>>(
            points, g, w.cell_start, w.vals, w.retry, f[F_RETRY], w.lists, w.big_lists, bcap, w.big_slot, w.counts,
            w.retry, w.fails, n, nullptr, nullptr, 0u);
        VT_LAUNCH_CHECK("voronoi_cells_kernel (large)");
    }
    rc = exclusive_scan_u32(w.counts, offsets, n + 1, w.scan_ws, s);
    if (rc)
        return rc;
    uint32_t tail[1 + F_WORDS];
    VT_HIP_CHECK(hipMemcpyAsync(tail, offsets + n, sizeof(uint32_t), hipMemcpyDeviceToHost, s));
    VT_HIP_CHECK(hipMemcpyAsync(tail + 1, w.fails, F_WORDS * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
    VT_HIP_CHECK(hipStreamSynchronize(s));
    if (tail[1 + F_FULL] || tail[1 + F_DEGENERATE]) {
        set_error("Voronoi build failed for %u cells over capacity (%d planes, %d vertices, %u lists longer than %d) "
                  "and %u degenerate cuts; first failing site %u; full tables (1 planes, 2 edges, 4 vertices, "
                  "8 lists): %u",
                  tail[1 + F_FULL], VorLarge::P, VorLarge::T, bcap, LIST_K, tail[1 + F_DEGENERATE],
                  tail[1 + F_FIRST_BAD], tail[1 + F_REASON]);
        return VT_ERR_INVALID;
    }
    *num_adjacency = tail[0];
    return VT_OK;
}

extern "C" int vt_voronoi_adjacency(uint32_t num_points, const uint32_t *offsets, uint32_t *adjacency,
                                    const void *workspace, vt_stream_t stream)
{
    clear_error();
    VT_REQUIRE(offsets && adjacency && workspace, "null pointer argument");
    hipStream_t s = as_stream(stream);
    VorWs w{};
    ws_words(num_points, &w, reinterpret_cast<uint32_t *>(const_cast<void *>(workspace)));
    voronoi_copy_kernel<<<(num_points + 255) / 256, 256, 0, s>>>(num_points, offsets, w.lists, w.big_lists,
                                                                 w.big_slot, adjacency);
    VT_LAUNCH_CHECK("voronoi_copy_kernel");
    return VT_OK;
}
