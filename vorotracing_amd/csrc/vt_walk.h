// vt_walk.h -- the Voronoi cell walk (tracing_octmap.cu:39-123) and the
// lane -> ray mapping of the traversal launches.
#pragma once

#include "vt_device.h"

namespace vt {

// The cell walk.  Starting in `start` at t0 = 0, each step searches the
// cell's face list for the nearest bisector plane with n.d > 0 (lowest face
// index wins ties), hands the segment [t0, t1) to the integrator when
// t1 > t0, and moves to the neighbour behind that face.  Faces are read in
// chunks of CHUNK records; records past the list end stay inside the 32-row
// padding and are masked, so the choice does not depend on CHUNK.  Returns the
// reference's step count n (the breaking iteration included).
template <int CHUNK, class Integrator, class StatsT>
__device__ __forceinline__ uint32_t walk(f3 o, f3 d, const float *__restrict__ points,
                                         const uint32_t *__restrict__ adjacency,
                                         const uint32_t *__restrict__ offsets, const uint2 *__restrict__ adj_diff,
                                         uint32_t start, uint32_t max_steps, Integrator &integ, StatsT &st)
{
    float t0 = 0.0f;
    uint32_t n = 0;
    uint32_t cur = start;
    f3 p = load_site(points, cur);
    for (;;) {
        n++;
        if (n > max_steps)
            break;
        uint32_t b = offsets[cur];
        uint32_t e = offsets[cur + 1];
        uint32_t nf = e - b;
        st.visit(cur, nf);
        float t1 = __builtin_huge_valf();
        uint32_t best = NONE;
        for (uint32_t i = 0; i < nf; i += CHUNK) {
            f3 off[CHUNK];
#pragma unroll
            for (int j = 0; j < CHUNK; ++j)
                off[j] = load_face(adj_diff, b + i + j);
#pragma unroll
            for (int j = 0; j < CHUNK; ++j) {
                f3 fo = mk(p.x + off[j].x * 0.5f, p.y + off[j].y * 0.5f, p.z + off[j].z * 0.5f);
                float dp = dot(off[j], d);
                float t = dot(sub(fo, o), off[j]) / dp;
                if (dp > 0.0f && t < t1 && (i + j) < nf) {
                    t1 = t;
                    best = i + j;
                }
            }
        }
        if (best == NONE)
            break;
        st.exit();
        uint32_t nxt = adjacency[b + best];
        f3 np = load_site(points, nxt);
        if (t1 > t0) {
            st.integrate();
            if (!integ.integrate(cur, t0, t1, p, np, st))
                break;
        }
        t0 = __builtin_fmaxf(t0, t1);
        cur = nxt;
        p = np;
    }
    return n;
}

// Lane -> ray for a tiled image batch: one wave (64 lanes) per tile_w x
// tile_h screen tile.  Returns NONE for lanes past the image edge.
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
    uint32_t y = (ti / tiles_x) * th + within / tw;
    uint32_t x = (ti % tiles_x) * tw + within % tw;
    if (img >= num_images || x >= W || y >= H)
        return NONE;
    return (img * H + y) * W + x;
}

} // namespace vt
