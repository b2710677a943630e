/*
 * oracle.h -- CPU restatement of the VoroTracing traversal hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py load it.  The
 * product library (vorotracing_amd/, libvt_hip.so) never links, loads or
 * calls it, and has no CPU fallback.
 *
 * Every entry point restates the reference arithmetic op for op (citations
 * are to /root/reference, see oracle.c).  The arithmetic convention shared by
 * restatement with the HIP kernels is:
 *   - dot(a, b) = fma(a2, b2, fma(a1, b1, a0 * b0))   (Eigen's a0b0+a1b1+a2b2
 *     as nvcc -O3 contracts it);
 *   - every other "a * b + c" the reference writes is fma(a, b, c); nothing
 *     else is contracted (-ffp-contract=off);
 *   - division and sqrt are IEEE correctly rounded;
 *   - exp/log are or_expf/or_logf (Cody-Waite reduction + Taylor / atanh
 *     series), f32<->f16 is round-to-nearest-even.
 * With that convention the GPU forward results are expected bit-identical.
 */
#ifndef VT_ORACLE_H
#define VT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Per-ray walk statistics; same layout as vt_ray_stats in include/vt_abi.h
 * (OR_STATS_LOG = VT_STATS_LOG). */
#define OR_STATS_LOG 24
typedef struct or_ray_stats {
    uint32_t n;          /* value returned by the walk */
    uint32_t visits;     /* cells whose face list was searched */
    uint32_t faces;      /* face records read */
    uint32_t exits;      /* exit faces found (neighbour id + next site read) */
    uint32_t integrated; /* integrate_cell calls (t1 > t0) */
    uint32_t shaded;     /* cells whose textures were fetched */
    uint64_t visit_hash; /* FNV-1a 64 over the visited cell ids */
    uint32_t first_cells[OR_STATS_LOG]; /* visited cells in walk order; 0xffffffff past the walk's end */
} or_ray_stats;

/* scalar helpers, exported so tests can pin them */
/* Planted mistakes, for the pin tests only: a test switches one on to show
 * that its check fails on that slip, then switches it back to 0 (none).  The
 * switch is process-wide and read during each call. */
enum {
    OR_PLANT_NONE = 0,
    OR_PLANT_SPEC_PLUS_D = 1,      /* specular sampled at oct_encode(+d), not (-d) */
    OR_PLANT_INFER_NO_DENSITY_GATE = 2, /* inference updates T for density <= 1e-6 */
    OR_PLANT_SKIP_ON_ALPHA = 3,    /* inference skip gate tests alpha, not the weight */
    OR_PLANT_NO_FIRST_CELL_TERM = 4,    /* backward: first cell's t0 term against the zero site dropped */
    OR_PLANT_FLUSH_CUR_ON_STOP = 5,     /* backward: opacity stop also flushes the next site's slot */
    OR_PLANT_POINT_ERROR_ALPHA = 6,     /* backward: point_error accumulates alpha * error */
    OR_PLANT_IGNORE_CONTRIB_GRAD = 7,   /* backward: contribution_alpha_grad not added */
    OR_PLANT_NO_DT0_PREV = 8            /* backward: previous site's t0 term dropped */
};
void or_set_plant(int code);
int or_get_plant(void);

/* Absolute-sum mode: while on, every atomically accumulated output (the
 * training backward's gradients, point_error, the forward's contribution)
 * adds |v| instead of v, so a call returns per element the sum of the
 * magnitudes scattered into it.  That sum bounds how far two summation
 * orders of the element can differ (the conditioning of the sum); the
 * parity tests scale their per-element tolerance by it.  With on = 2 every
 * add adds 1 instead: the number of adds per element, which bounds the
 * rounding of sums kept in half precision (one rounding per add).  Off (0) in
 * every other use. */
void or_set_abs_sums(int on);

float or_expf(float x);
float or_logf(float x);
uint16_t or_f32_to_f16(float x);
float or_f16_to_f32(uint16_t h);
void or_expf_many(const float *x, float *y, size_t n);
void or_logf_many(const float *x, float *y, size_t n);
void or_f32_to_f16_many(const float *x, uint16_t *y, size_t n);
/* the walk's exit-face search on rows of 26 floats (site, origin, direction,
 * face count as u32 bits, 8 half4 records); out: face index, t1 bits */
void or_exit_face_many(const float *rows, size_t n, uint32_t *out);
int or_oct_wrap_index(int u, int v, int R);
void or_oct_encode(const float dir[3], int R, float uv[2]);

/* Camera ray generation (the rays the reference builds in torch:
 * utils/__init__.py:85-130, datasets/datasets.py:126-136 and :286-304; the
 * fisheye model is OpenCV's, which the reference reaches through pycolmap's
 * cam_from_img).  Same layout and semantics as vt_camera in
 * include/vt_abi.h. */
enum { OR_CAMERA_PINHOLE = 0, OR_CAMERA_FISHEYE = 1 };
typedef struct or_camera {
    uint32_t model;
    float fx, fy, cx, cy;
    float pixel_offset;
    float k[4];
    float R[9];
    float t[3];
    float rolling[3];
} or_camera;
float or_sinf(float x); /* x in [0, pi] */
float or_cosf(float x); /* x in [0, pi] */
void or_sincos_many(int cos, const float *x, float *y, size_t n);
/* rays f32 (num_images, H, W, 6); direction not normalised (the walk does). */
void or_camera_rays(const or_camera *cams, uint32_t num_images, uint32_t H, uint32_t W, float *rays);

/* tracing_octmap.cu:125-149; adj_diff has (adjacency_size + 32) * 4 halves,
 * the 32-row tail is left untouched (uninitialised in the reference). */
void or_prefetch_adj(const float *points, uint32_t num_points, const uint32_t *adjacency,
                     const uint32_t *offsets, uint16_t *adj_diff, int num_threads);

/* tracing_octmap.cu:552-610 (fp16 inference).  diffuse/specular are
 * Half4Texel maps (N, 4*R*R) halves.  ray_perm may be NULL.  visits_out (if
 * not NULL) receives the first max_log visited cells of each ray (rest filled
 * with 0xffffffff). */
void or_trace_infer_f16(const float *points, const uint16_t *diffuse, const uint16_t *specular,
                        int diff_res, int spec_res, const float *density, const uint32_t *adjacency,
                        const uint32_t *offsets, const uint16_t *adj_diff, const float *rays,
                        uint32_t num_rays, const uint32_t *start_point, const uint32_t *ray_perm,
                        float weight_threshold, uint32_t max_intersections, float cell_skip_threshold,
                        uint16_t *rgba, or_ray_stats *stats, uint32_t *visits_out, uint32_t max_log,
                        int num_threads);

/* tracing_octmap.cu:723-779 (q8 inference).  u8 maps (N, 3*R*R); per-channel
 * scale/offset (the reference's per-tensor pair is the case of 3 equal
 * values). */
void or_trace_infer_q8(const float *points, const uint8_t *diffuse, const uint8_t *specular,
                       int diff_res, int spec_res, const float diff_scale[3], const float diff_offset[3],
                       const float spec_scale[3], const float spec_offset[3], const float *density,
                       const uint32_t *adjacency, const uint32_t *offsets, const uint16_t *adj_diff,
                       const float *rays, uint32_t num_rays, const uint32_t *start_point,
                       float weight_threshold, uint32_t max_intersections, float cell_skip_threshold,
                       uint16_t *rgba, or_ray_stats *stats, int num_threads);

/* tracing_octmap.cu:151-230 + host :346-546 (training forward).  attr_f16 = 0
 * for float32 maps/rgba/contribution, 1 for float16.  depth, depth_idx,
 * contribution, n may be NULL as in the reference.  adj_diff must be the
 * prefetch output for the same scene. */
void or_trace_fwd(int attr_f16, const float *points, const void *diffuse, const void *specular,
                  int diff_res, int spec_res, const float *density, const uint32_t *adjacency,
                  const uint32_t *offsets, const uint16_t *adj_diff, const float *rays, uint32_t num_rays,
                  const uint32_t *start_point, uint32_t num_quantiles, const float *depth_quantiles,
                  float weight_threshold, uint32_t max_intersections, void *rgba, float *depth,
                  uint32_t *depth_idx, void *contribution, uint32_t *num_intersections, float *distortion,
                  float *W_total, float *S_total, float *t_far, or_ray_stats *stats, int num_threads);

/* tracing_octmap.cu:232-340 + host :860-1103 (training backward).  Output
 * gradient buffers must be zeroed by the caller.  depth_quantiles,
 * depth_idx, depth_grad, ray_error, distortion_grad, point_error may be NULL. */
void or_trace_bwd(int attr_f16, const float *points, const void *diffuse, const void *specular,
                  int diff_res, int spec_res, const float *density, const uint32_t *adjacency,
                  const uint32_t *offsets, const uint16_t *adj_diff, const float *rays, uint32_t num_rays,
                  const uint32_t *start_point, const void *rgba, const void *rgba_grad,
                  uint32_t num_quantiles, const float *depth_quantiles, const uint32_t *depth_idx,
                  const float *depth_grad, const void *ray_error, float contribution_alpha_grad,
                  const float *distortion, const float *distortion_grad, const float *W_total,
                  const float *S_total, const float *t_far, float weight_threshold,
                  uint32_t max_intersections, float *points_grad, void *diffuse_grad, void *specular_grad,
                  float *density_grad, void *point_error, or_ray_stats *stats, int num_threads);

/* Exact nearest site per query (what NNBVH.query returns, nn_bvh.cu:29-41):
 * fp32 squared distance dot(q-p, q-p), ties -> lowest index.  int32 out. */
void or_nearest_site(const float *points, uint32_t num_points, const float *queries, uint32_t num_queries,
                     int32_t *out, int num_threads);

/* d t / d prim for the bisector plane of (prim, opp) (ray_integrator.cuh:39-53) */
void or_cell_intersection_grad(const float prim[3], const float opp[3], const float o[3], const float d[3],
                               float out[3]);

#ifdef __cplusplus
}
#endif
#endif
