/*
 * vt_abi.h -- C ABI of libvt_hip.so, the MI355X (gfx950) VoroTracing
 * traversal library.
 *
 * Plain pointers and sizes only.  All array arguments are device pointers
 * (HBM), contiguous, in the reference layouts noted per function.  `stream`
 * is a hipStream_t (NULL = the null stream).  Every entry returns 0 on
 * success or a VT_ERR_* code; vt_last_error() returns the calling thread's
 * last message.  Entries enqueue work on `stream` and do not synchronise.
 *
 * Reference citations are to zenseact/VoroTracing (vorotracing/cuda/csrc).
 */
#ifndef VT_ABI_H
#define VT_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *vt_stream_t;

enum {
    VT_OK = 0,
    VT_ERR_INVALID = 1,     /* bad argument (message names it) */
    VT_ERR_HIP = 2,         /* HIP runtime / launch error */
    VT_ERR_UNSUPPORTED = 3, /* e.g. texture resolution not compiled */
    VT_ERR_NOMEM = 4
};

enum { VT_ATTR_F32 = 0, VT_ATTR_F16 = 1 };

/* Per-ray walk statistics (debug / roofline accounting).  Filled only when a
 * non-NULL `stats` array (one record per ray, in ray order) is passed.  The
 * first VT_STATS_LOG visited cells locate the first step at which two walks
 * part; the hash covers the whole walk.  128 bytes per ray. */
#define VT_STATS_LOG 24
typedef struct vt_ray_stats {
    uint32_t n;          /* value returned by the walk (trace_octmap) */
    uint32_t visits;     /* cells whose face list was searched */
    uint32_t faces;      /* face records read */
    uint32_t exits;      /* exit faces found (neighbour id + next site read) */
    uint32_t integrated; /* integrate_cell calls (t1 > t0) */
    uint32_t shaded;     /* cells whose textures were fetched */
    uint64_t visit_hash; /* FNV-1a 64 over the visited cell ids */
    uint32_t first_cells[VT_STATS_LOG]; /* visited cells in walk order; 0xffffffff past the walk's end */
} vt_ray_stats;

/* Message of the calling thread's last failed call ("" if none). */
const char *vt_last_error(void);
/* ABI version (bumped on incompatible change). */
int vt_abi_version(void);

/*
 * Prefetch of per-face site offsets.  Replaces _C.trace_vorotracing_prefetch_adj
 * (tracing_octmap.cu:612-640, kernel :125-149).
 *   points (num_points,3) f32; adjacency u32 (adjacency_size, including the
 *   32-entry padding); offsets u32 (num_points+1).
 *   adj_diff out: f16 (adjacency_size+32, 4) = half(site[adj[e]] - site[i]), w = 0.
 *   Rows past offsets[num_points] are zero-filled.
 */
int vt_prefetch_adj(const float *points, uint32_t num_points, const uint32_t *adjacency, uint32_t adjacency_size,
                    const uint32_t *offsets, uint16_t *adj_diff, vt_stream_t stream);

/*
 * Packed walk layout (extension; no counterpart in the reference).  The
 * scene's face records regrouped so that a traversal step issues fewer
 * vector loads, which bound the traversal kernels:
 *   chunks: u32 (num_chunks + 1, 12).  Each cell's face list in chunks of 8
 *     faces, 24 halves each: x, y, z of the chunk's first face, then of its
 *     second, ... (the adj_diff halves).  A list is padded to a multiple of 8
 *     with zero offsets, never an exit face (n.d = 0).  The walk loads a
 *     cell's first chunk before it knows the list is not empty, so the array
 *     holds one chunk more (any contents).
 *   links: u32 (8 * num_chunks, 2).  Per padded face slot k of cell c, at
 *     8 * first_chunk[c] + k: {neighbour | its chunk count << 24, its first
 *     chunk}.
 *   heads: u32 (num_points, 2): the same pair for each cell itself.
 *   cells: f32 (num_points, 4): {site xyz, density}.
 *   orig: u16 (8 * num_chunks): each slot's index in the cell's original
 *     list (0xffff for pads).  A list of at most 64 faces is laid out in the
 *     order of one component of its offsets (face_order 1, 2, 3: x, y, z;
 *     0 keeps the list order), compared as f16 values with -0 taken as +0
 *     and NaNs past the infinities of their sign, equal values in list
 *     order: the lanes of a
 *     wave, whose rays point alike, then meet forward-facing faces at the same
 *     slots, and the wave skips the plane test of slots that no lane faces.
 *     Quotients that tie go to the lower original index, as in the reference.
 * The walk reads the same offsets, sites and densities as through adjacency,
 * offsets and adj_diff and picks the same exit faces, so it renders the same
 * images bit for bit.  Limits:
 * num_points < 2^24, at most 255 chunks (2,040 faces) per cell and
 * 8 * num_chunks < 2^32.
 */
typedef struct vt_walk_layout {
    const uint32_t *chunks;
    const uint32_t *links;
    const uint32_t *heads;
    const float *cells;
    const uint16_t *orig;
    uint32_t num_chunks;
} vt_walk_layout;

/* Bytes of workspace for vt_walk_layout_count. */
size_t vt_walk_layout_count_workspace_size(uint32_t num_points);
/*
 * Chunk ranges of the layout.  first_chunk out: u32 (num_points + 2):
 * first_chunk[c] = chunks of the cells before c, [num_points] = the total
 * (num_chunks), [num_points + 1] = the largest chunk count of one cell, with
 * bit 31 set when an adjacency entry is num_points or more; the caller checks
 * the limits and the flag on the last two before vt_walk_layout_fill (which
 * links a cell to itself in place of such an entry, and never reads out of
 * bounds).
 */
int vt_walk_layout_count(const uint32_t *offsets, const uint32_t *adjacency, uint32_t num_points,
                         uint32_t *first_chunk, void *ws, vt_stream_t stream);
/*
 * Fill the layout (arrays sized for num_chunks = first_chunk[num_points]).
 * density: the f32 per-cell density the renders integrate; adj_diff from
 * vt_prefetch_adj.
 */
int vt_walk_layout_fill(const float *points, const float *density, const uint32_t *adjacency,
                        const uint32_t *offsets, uint32_t num_points, const uint16_t *adj_diff,
                        const uint32_t *first_chunk, uint32_t num_chunks, int face_order, uint32_t *chunks,
                        uint32_t *links, uint32_t *heads, float *cells, uint16_t *orig, vt_stream_t stream);

/*
 * Footprint tables of octahedral maps (extension; no counterpart in the
 * reference: a layout of the maps that the tiled and camera inference entries
 * can read in place of the maps' texels).  For maps of res x res texels
 * (res 4 or 8), a cell's table has (res + 1)^2 entries.  Entry
 * ey * (res + 1) + ex holds the four texels that a bilinear tap with floor
 * coordinates (ex - 1, ey - 1) reads, at (ex - 1, ey - 1), (ex, ey - 1),
 * (ex - 1, ey) and (ex, ey), each through the octahedral wrap
 * (oct_wrap_index, ray_integrator_octmap.cuh:36-55), with the same texels and
 * weights as the maps: the images are the same bit for bit.
 *   fp16 (vt_quad_maps_f16): maps Half4Texel f16 (num_points, 4 * res * res);
 *   quads out f16 (num_points, 16 * (res + 1)^2): 32-byte entries, two
 *   16-byte loads per tap in one cache line instead of four 8-byte texels.
 *   q8 (vt_quad_maps_q8): maps u8 (num_points, 3 * res * res); quads out u8
 *   (num_points, 16 * (res + 1)^2): 16-byte entries of four (r, g, b, 0)
 *   texels, one load per tap instead of twelve single bytes.
 * quads is 16-byte aligned.
 */
enum { VT_QUAD_F16 = 0, VT_QUAD_Q8 = 1 };
typedef struct vt_quad_maps {
    const void *diffuse;  /* table of the diffuse map (diff_res) */
    const void *specular; /* table of the specular map (spec_res) */
    uint32_t num_points;  /* cells of the tables; a render checks them */
    uint32_t diff_res;    /* against its num_points, diff_res and */
    uint32_t spec_res;    /* spec_res */
    uint32_t format;      /* VT_QUAD_F16 or VT_QUAD_Q8, checked against the entry */
} vt_quad_maps;

int vt_quad_maps_f16(const uint16_t *maps, uint32_t num_points, uint32_t res, uint16_t *quads, vt_stream_t stream);
int vt_quad_maps_q8(const uint8_t *maps, uint32_t num_points, uint32_t res, uint8_t *quads, vt_stream_t stream);

/*
 * fp16 inference render.  Replaces _C.trace_vorotracing_infer
 * (tracing_octmap.cu:642-717, kernel :552-610).
 *   diffuse/specular: Half4Texel maps, f16 (num_points, 4*R*R), R = diff_res /
 *   spec_res in {4, 8}.  density f32 (num_points).  adj_diff from
 *   vt_prefetch_adj.  rays f32 (num_rays, 6).  start_point u32 (num_rays).
 *   ray_perm u32 (num_rays) or NULL: lane t renders ray ray_perm[t].
 *   rgba out: f16 (num_rays, 4) in ray order.  stats: NULL or (num_rays).
 * A start cell at or past num_points (which the reference would read out of
 * bounds) gives its ray no step: rgba (0, 0, 0, 0), n = 0.  This holds for
 * every inference and training entry; the other rays are unchanged.
 */
int vt_trace_infer_f16(const float *points, const uint16_t *diffuse, const uint16_t *specular, uint32_t diff_res,
                       uint32_t spec_res, const float *density, const uint32_t *adjacency, const uint32_t *offsets,
                       uint32_t num_points, const uint16_t *adj_diff, const float *rays, uint32_t num_rays,
                       const uint32_t *start_point, const uint32_t *ray_perm, float weight_threshold,
                       uint32_t max_intersections, float cell_skip_threshold, uint16_t *rgba, vt_ray_stats *stats,
                       vt_stream_t stream);

/*
 * fp16 inference over image batches with in-kernel wave tiling: rays are
 * (num_images, image_h, image_w, 6) and each 64-lane wave renders one
 * tile_w x tile_h screen tile (tile_w * tile_h == 64), so no permutation
 * buffer is read.  Results are identical to vt_trace_infer_f16 (the lane
 * assignment never changes per-ray results, vorotracing.py:606-625).
 * tile_order: NULL (tiles in screen order) or the launch order of the
 * ceil(W/tile_w) * ceil(H/tile_h) * num_images tiles (vt_tile_order);
 * tile_cost: NULL or one u32 per tile, written with each tile's cost for
 * vt_tile_order (both extensions).  rays_per_start: 0 when start_point holds
 * one cell per ray, else the number of consecutive rays that share one start
 * cell (ray r starts at start_point[r / rays_per_start]; H * W for one cell
 * per pinhole image; extension).  walk: NULL, or the scene's packed walk
 * layout (vt_walk_layout; extension), which the kernel then walks in place of
 * adjacency / adj_diff (same results; offsets still serve stats).  quads:
 * NULL, or the footprint tables of the two maps (vt_quad_maps; extension),
 * which the kernel then reads in place of the maps' texels (same results).
 */
int vt_trace_infer_f16_tiled(const float *points, const uint16_t *diffuse, const uint16_t *specular,
                             uint32_t diff_res, uint32_t spec_res, const float *density, const uint32_t *adjacency,
                             const uint32_t *offsets, uint32_t num_points, const uint16_t *adj_diff,
                             const float *rays, uint32_t num_images, uint32_t image_h, uint32_t image_w,
                             uint32_t tile_h, uint32_t tile_w, const uint32_t *start_point, uint32_t rays_per_start,
                             float weight_threshold,
                             uint32_t max_intersections, float cell_skip_threshold, uint16_t *rgba,
                             const uint32_t *tile_order, uint32_t *tile_cost, vt_ray_stats *stats,
                             const vt_walk_layout *walk, const vt_quad_maps *quads, vt_stream_t stream);

/*
 * q8 inference render.  Replaces _C.trace_vorotracing_infer_q8
 * (tracing_octmap.cu:781-854, kernel :723-779).
 *   diffuse/specular u8 (num_points, 3*R*R); dequant = scale[c]*q + offset[c]
 *   per RGB channel c (the reference's per-tensor pair = 3 equal values).
 *   ray_perm: u32 or NULL (the reference has none; NULL reproduces it).
 */
int vt_trace_infer_q8(const float *points, const uint8_t *diffuse, const uint8_t *specular, uint32_t diff_res,
                      uint32_t spec_res, const float diff_scale[3], const float diff_offset[3],
                      const float spec_scale[3], const float spec_offset[3], const float *density,
                      const uint32_t *adjacency, const uint32_t *offsets, uint32_t num_points,
                      const uint16_t *adj_diff, const float *rays, uint32_t num_rays, const uint32_t *start_point,
                      const uint32_t *ray_perm, float weight_threshold, uint32_t max_intersections,
                      float cell_skip_threshold, uint16_t *rgba, vt_ray_stats *stats, vt_stream_t stream);

/*
 * q8 inference over image batches with in-kernel wave tiling (as
 * vt_trace_infer_f16_tiled, walk and quads (q8 tables) included; per-ray
 * results identical to vt_trace_infer_q8).
 */
int vt_trace_infer_q8_tiled(const float *points, const uint8_t *diffuse, const uint8_t *specular, uint32_t diff_res,
                            uint32_t spec_res, const float diff_scale[3], const float diff_offset[3],
                            const float spec_scale[3], const float spec_offset[3], const float *density,
                            const uint32_t *adjacency, const uint32_t *offsets, uint32_t num_points,
                            const uint16_t *adj_diff, const float *rays, uint32_t num_images, uint32_t image_h,
                            uint32_t image_w, uint32_t tile_h, uint32_t tile_w, const uint32_t *start_point,
                            uint32_t rays_per_start, float weight_threshold, uint32_t max_intersections,
                            float cell_skip_threshold,
                            uint16_t *rgba, const uint32_t *tile_order, uint32_t *tile_cost, vt_ray_stats *stats,
                            const vt_walk_layout *walk, const vt_quad_maps *quads, vt_stream_t stream);

/*
 * Cameras for in-kernel ray generation.  Replaces the rays buffer that the
 * reference builds in torch before every render: vorotracing/utils/
 * __init__.py:85-130 (generate_camera_rays) and datasets/datasets.py:126-136,
 * :286-304 (pixel centres, cam_from_img, normalise, rotate by the pose).
 * Pixel (u, v) of an H x W image samples (u + pixel_offset, v + pixel_offset)
 * (datasets.py uses 0.5, generate_camera_rays 0):
 *   mx = (u + pixel_offset - cx) / fx,  my = (v + pixel_offset - cy) / fy
 *   pinhole: dir_cam = (mx, my, 1)
 *   fisheye (OpenCV fisheye / equidistant): theta_d = |(mx, my)|, theta solves
 *     theta (1 + k1 theta^2 + k2 theta^4 + k3 theta^6 + k4 theta^8) = theta_d
 *     (12 Newton steps from theta_d, clamped to [0, pi]),
 *     dir_cam = (mx sin(theta) / theta_d, my sin(theta) / theta_d, cos(theta))
 *   dir_cam /= |dir_cam|; ray direction = R dir_cam (R row-major,
 *   camera-to-world; the traversal normalises it again as it does any ray);
 *   origin = t + (v / (H - 1)) * rolling (rolling shutter; zero for a
 *   global shutter).
 * The arithmetic is f32 with the library's convention (fused dot products,
 * correctly rounded division and sqrt, own sin / cos polynomials).
 */
enum { VT_CAMERA_PINHOLE = 0, VT_CAMERA_FISHEYE = 1 }; /* other values render as pinhole */
typedef struct vt_camera {
    uint32_t model;     /* VT_CAMERA_* */
    float fx, fy, cx, cy;
    float pixel_offset;
    float k[4];         /* fisheye distortion k1..k4 */
    float R[9];         /* camera-to-world rotation, row-major */
    float t[3];         /* camera centre */
    float rolling[3];   /* origin shift at the last row */
} vt_camera;

/*
 * Rays of num_images cameras (device array) for H x W images, written as
 * f32 (num_images, H, W, 6): the rays the camera renders below trace.
 * With W = 1 the origins are those of each row (start cells of
 * rolling-shutter cameras).
 */
int vt_camera_rays(const vt_camera *cameras, uint32_t num_images, uint32_t image_h, uint32_t image_w, float *rays,
                   vt_stream_t stream);

/*
 * fp16 / q8 inference of num_images cameras (device array), rays generated in
 * the kernel: no rays buffer is read.  Per-ray results equal those of
 * vt_trace_infer_f16_tiled / vt_trace_infer_q8_tiled on the rays of
 * vt_camera_rays.  start_point: u32 start cell per image, or per image row
 * ((num_images, image_h)) when start_per_row is non-zero (rolling shutter:
 * every row has its own origin).  rgba (num_images, image_h, image_w, 4) f16;
 * stats in the same ray order.  walk and quads: as for
 * vt_trace_infer_f16_tiled (quads of the entry's format).
 */
int vt_trace_infer_f16_camera(const float *points, const uint16_t *diffuse, const uint16_t *specular,
                              uint32_t diff_res, uint32_t spec_res, const float *density, const uint32_t *adjacency,
                              const uint32_t *offsets, uint32_t num_points, const uint16_t *adj_diff,
                              const vt_camera *cameras, uint32_t num_images, uint32_t image_h, uint32_t image_w,
                              uint32_t tile_h, uint32_t tile_w, const uint32_t *start_point, int start_per_row,
                              float weight_threshold, uint32_t max_intersections, float cell_skip_threshold,
                              uint16_t *rgba, const uint32_t *tile_order, uint32_t *tile_cost, vt_ray_stats *stats,
                              const vt_walk_layout *walk, const vt_quad_maps *quads, vt_stream_t stream);
int vt_trace_infer_q8_camera(const float *points, const uint8_t *diffuse, const uint8_t *specular, uint32_t diff_res,
                             uint32_t spec_res, const float diff_scale[3], const float diff_offset[3],
                             const float spec_scale[3], const float spec_offset[3], const float *density,
                             const uint32_t *adjacency, const uint32_t *offsets, uint32_t num_points,
                             const uint16_t *adj_diff, const vt_camera *cameras, uint32_t num_images,
                             uint32_t image_h, uint32_t image_w, uint32_t tile_h, uint32_t tile_w,
                             const uint32_t *start_point, int start_per_row, float weight_threshold,
                             uint32_t max_intersections, float cell_skip_threshold, uint16_t *rgba,
                             const uint32_t *tile_order, uint32_t *tile_cost, vt_ray_stats *stats,
                             const vt_walk_layout *walk, const vt_quad_maps *quads, vt_stream_t stream);

/*
 * Training forward.  Replaces _C.trace_vorotracing_fwd
 * (tracing_octmap.cu:346-546, kernel :151-230).  Runs the prefetch into
 * `adj_diff_workspace` ((adjacency_size+32)*4 halves) as the reference does
 * on every call, then the traversal.
 *   attr_dtype VT_ATTR_F32 / VT_ATTR_F16 for diffuse/specular (num_points,
 *   3*R*R), rgba (num_rays,4) and contribution (num_points).
 *   depth_quantiles f32 (num_rays, K) or NULL (K ignored); depth f32 and
 *   depth_idx u32 (num_rays, K) outputs when quantiles are given.
 *   contribution: NULL or zero-initialised (num_points), accumulated.
 *   num_intersections u32, distortion/W_total/S_total/t_far f32 (num_rays).
 *   image_h, image_w: lane order only.  When both are non-zero and
 *   image_h*image_w divides num_rays, the rays are row-major images of that
 *   size and each wave traces one 8x8 screen tile (neighbouring rays share
 *   cells, so same-cell gradient combining finds more partners); 0, 0 = ray
 *   order.  Outputs do not depend on it beyond the order of atomic adds.
 *   ray_perm: u32 (num_rays) lane order or NULL (an extension, ABI version
 *   5): lane t traces ray ray_perm[t], overriding image_h/image_w; it must
 *   be a permutation of 0..num_rays-1 (an entry >= num_rays leaves its
 *   lane idle).  vt_ray_order makes one for flat batches.
 *   tile_order, tile_cost (extensions, ABI versions 9-10): with image lanes
 *   (tiles: screen tiles) or a ray_perm (tiles: waves of 64 consecutive
 *   ray_perm entries, a half-wave taking 32 of them),
 *   NULL or the tiles + 1 words of vt_tile_order (split_waves =
 *   vt_train_fwd_resident_waves()) over the costs a forward of the same rays
 *   recorded, and NULL or one u32 per tile receiving each tile's cost for
 *   vt_tile_order, as for the tiled inference entries.  Given an order with a
 *   non-zero split count, the launch takes the tiles in that order and runs
 *   the first tile_order[tiles] as two half-waves each (rows 0-3, rows 4-7);
 *   a split tile's cost is then the larger of its halves' costs (each
 *   half's longest walk and most face records), recorded with an atomic max:
 *   clear tile_cost before such a call.  With a split count of 0 the order
 *   is ignored (screen order).
 */
int vt_trace_fwd(int attr_dtype, const float *points, const void *diffuse, const void *specular, uint32_t diff_res,
                 uint32_t spec_res, const float *density, const uint32_t *adjacency, uint32_t adjacency_size,
                 const uint32_t *offsets, uint32_t num_points, const float *rays, uint32_t num_rays,
                 uint32_t image_h, uint32_t image_w, const uint32_t *start_point, const uint32_t *ray_perm,
                 uint32_t num_quantiles, const float *depth_quantiles,
                 float weight_threshold, uint32_t max_intersections, void *rgba, float *depth, uint32_t *depth_idx,
                 void *contribution, uint32_t *num_intersections, float *distortion, float *W_total,
                 float *S_total, float *t_far, uint16_t *adj_diff_workspace, const uint32_t *tile_order,
                 uint32_t *tile_cost, vt_ray_stats *stats, vt_stream_t stream);

/*
 * Training backward.  Replaces _C.trace_vorotracing_bwd
 * (tracing_octmap.cu:860-1103, kernel :232-340).  Prefetch into the
 * workspace as in vt_trace_fwd, then the re-walk with gradient scatter.
 *   adj_diff_ready (an extension, ABI version 6): 0 = prefetch as the
 *   reference does; 1 = adj_diff_workspace already holds the prefetch of
 *   these points and adjacency (the forward of the same call filled it and
 *   neither has changed since), which the call then skips.
 *   rgba / rgba_grad: attr dtype (num_rays, 4).  depth_quantiles, depth_idx,
 *   depth_grad (num_rays, K) or NULL.  ray_error: attr dtype (num_rays) or
 *   NULL.  distortion, W_total, S_total, t_far: f32 (num_rays);
 *   distortion_grad f32 (num_rays) or NULL.
 *   Outputs (caller zero-initialises): points_grad f32 (num_points,3),
 *   diffuse_grad / specular_grad attr dtype, density_grad f32 (num_points),
 *   point_error attr dtype (num_points) or NULL.
 *   image_h, image_w, ray_perm: lane order, as for vt_trace_fwd.
 *   cell_workspace: f32 (num_points, 4), 16-byte aligned, any contents (an
 *   extension, ABI version 4): the call accumulates each cell's point and
 *   density gradients there, in one 16-byte slot per cell, and adds the
 *   slots into points_grad and density_grad at its end.
 *   Gradient scatters of lanes that integrate the same cell in the same step
 *   are combined in LDS before the global atomics.
 *   tile_order (an extension, ABI version 10): with image lanes or a
 *   ray_perm (tiles as for vt_trace_fwd), NULL or the tiles + 1 words of
 *   vt_tile_order over the costs the forward of these rays recorded.  Tiles launch in that order, and the first
 *   tile_order[tiles] of them (at most vt_train_bwd_resident_waves()) run as
 *   two half-waves of 32 rays each.
 */
int vt_trace_bwd(int attr_dtype, const float *points, const void *diffuse, const void *specular, uint32_t diff_res,
                 uint32_t spec_res, const float *density, const uint32_t *adjacency, uint32_t adjacency_size,
                 const uint32_t *offsets, uint32_t num_points, const float *rays, uint32_t num_rays,
                 uint32_t image_h, uint32_t image_w, const uint32_t *start_point, const uint32_t *ray_perm,
                 const void *rgba, const void *rgba_grad, uint32_t num_quantiles,
                 const float *depth_quantiles, const uint32_t *depth_idx, const float *depth_grad,
                 const void *ray_error, float contribution_alpha_grad, const float *distortion,
                 const float *distortion_grad, const float *W_total, const float *S_total, const float *t_far,
                 float weight_threshold, uint32_t max_intersections, float *points_grad, void *diffuse_grad,
                 void *specular_grad, float *density_grad, void *point_error, uint16_t *adj_diff_workspace,
                 int adj_diff_ready, float *cell_workspace, const uint32_t *tile_order, vt_ray_stats *stats,
                 vt_stream_t stream);

/*
 * Coherent lane order for a flat training batch (an extension: the reference
 * traces rays in batch order, tracing_octmap.cu:175-179 and :264-268, and its default
 * trainer batches random pixels of random images, datasets.py:185-222 with
 * trainer.py:52).
 *   ray_perm (num_rays) u32 out: the rays sorted by start cell, then by a
 *   2-D Morton code of the direction's octahedral coordinates (a 128 x 128
 *   grid), stable, so that a wave traces rays of one camera with neighbouring
 *   directions.  Pass it as vt_trace_fwd / vt_trace_bwd's ray_perm.
 *   workspace: vt_ray_order_workspace_size(num_rays) bytes, 4-byte aligned.
 */
size_t vt_ray_order_workspace_size(uint32_t num_rays);
int vt_ray_order(const float *rays, const uint32_t *start_point, uint32_t num_rays, uint32_t num_points,
                 uint32_t *ray_perm, void *workspace, vt_stream_t stream);

/*
 * Start-cell lookup.  Replaces _C.NNBVH (nn_bvh.h:4-16, nn_bvh.cu:43-109):
 * a Morton LBVH built on the GPU, exact nearest-site queries.
 *   vt_bvh_create: new empty handle (host object owning device memory).
 *   vt_bvh_build: (re)build over points (num_points, 3) f32 (nn_bvh.cu:63-89).
 *   vt_bvh_query: out[i] = index of the site nearest to queries[i] (int32,
 *   nn_bvh.cu:91-109); squared distance in fp32, ties to the lowest index.
 *   `points` must be the array the handle was built on.  Up to 2^26
 *   query-site pairs (a frame's camera origins) a query scans all sites
 *   instead of walking the tree (same distances, same answer), keeping
 *   per-block partials in the handle's workspace: builds and queries of one
 *   handle must be ordered on one stream.
 *   vt_bvh_destroy: free the handle (nn_bvh.cu:53-61).
 */
int vt_bvh_create(void **handle);
int vt_bvh_destroy(void *handle);
int vt_bvh_build(void *handle, const float *points, uint32_t num_points, vt_stream_t stream);
int vt_bvh_query(void *handle, const float *points, uint32_t num_points, const float *queries, uint32_t num_queries,
                 int32_t *out, vt_stream_t stream);
int vt_bvh_num_nodes(void *handle);
/*
 * The query of vt_bvh_query (nn_bvh.cu:91-109) without the handle's
 * workspace: when the all-sites scan is the faster path (num_queries *
 * num_points <= VT_NN_SCAN_PAIRS and num_queries <= VT_NN_SCAN_MAX_QUERIES)
 * its per-block partials go in `workspace`
 * (8-byte aligned, vt_nearest_scan_workspace_size(num_queries) bytes; with
 * less, or NULL, the tree is walked).  The handle is only read, so queries of
 * one built handle may run on several streams at once.
 */
#define VT_NN_SCAN_PAIRS (1ull << 26)
#define VT_NN_SCAN_MAX_QUERIES 64
size_t vt_nearest_scan_workspace_size(uint32_t num_queries);
int vt_bvh_query_ws(void *handle, const float *points, uint32_t num_points, const float *queries, uint32_t num_queries,
                    int32_t *out, void *workspace, size_t workspace_bytes, vt_stream_t stream);
/*
 * Start cells of a ray batch: start[i] = the site nearest the origin of ray
 * i (rays (num_rays, 6) f32, origin first; the reference's per-ray query of
 * vorotracing.py:323-344, nn_bvh.cu:91-109), with the tree's distance and
 * tie rule.  One tree query per run of equal consecutive origins (a
 * camera's rays share one, a rolling shutter has one per row), counted and
 * compacted on the device, so the call never waits for the GPU (an
 * extension, ABI version 10).  workspace: vt_start_cells_workspace_size(
 * num_rays) bytes, 4-byte aligned.  The handle is only read.
 */
size_t vt_start_cells_workspace_size(uint32_t num_rays);
int vt_start_cells(void *handle, const float *points, uint32_t num_points, const float *rays, uint32_t num_rays,
                   uint32_t *start, void *workspace, vt_stream_t stream);
/* Test hook (no reference counterpart): caps the tree walk's stack at `limit`
 * entries (1..64; 0 restores 64) and, if force_tree, makes every query walk
 * the tree.  A query whose stack would overflow answers by a scan of all
 * sites (same distance and tie rule), so a capped stack reaches that path. */
int vt_bvh_debug_stack_limit(void *handle, uint32_t limit, int force_tree);

/*
 * Allocation-free nearest-site lookup.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops).  out[i] = index of the site nearest to
 * queries[i] (int32), the answer vt_bvh_query gives (squared distance in
 * fp32, ties to the lowest index), computed by a scan of all num_points sites
 * without a handle.  At most 64 queries per call (512 KiB of per-block
 * partials in a static device array that each GPU holds until the process
 * ends); more is rejected with VT_ERR_INVALID.  No hipMalloc or hipFree.
 * Every call on one GPU shares that array: calls that overlap on one GPU
 * (concurrent streams, threads) race; order them on one stream.  The first
 * call on a device looks up the array's address there (hipGetSymbolAddress);
 * a call with num_queries = 0 does only that, so a caller that captures the
 * lookup into a HIP graph makes one such call first, outside the capture.
 * Each call is then two kernel launches on `stream` and no memset.
 */
int vt_nearest_sites_noalloc(const float *points, uint32_t num_points, const float *queries, uint32_t num_queries,
                             int32_t *out, vt_stream_t stream);

/*
 * Morton reorder of cells.  Replaces VoroTracingInfer._reorder_by_morton
 * (vorotracing.py:514-571): 10-bit-per-axis Morton keys of the sites in their
 * bounding box, stable sort (the reference's argsort leaves ties unordered),
 * perm[i] = old index of new cell i, sites gathered, neighbour ids remapped,
 * face lists copied in their original order, new offsets; adjacency_out
 * (adjacency_size entries) is zero past offsets_out[num_points].
 * workspace: vt_morton_workspace_size() bytes.  Other per-cell rows
 * (density, textures) follow with vt_permute_rows.
 */
size_t vt_morton_workspace_size(uint32_t num_points, uint32_t adjacency_size);
int vt_morton_reorder(const float *points, uint32_t num_points, const uint32_t *adjacency, uint32_t adjacency_size,
                      const uint32_t *offsets, uint32_t *perm, float *points_out, uint32_t *adjacency_out,
                      uint32_t *offsets_out, void *workspace, vt_stream_t stream);
/* dst row i = src row perm[i] (rows of row_bytes bytes; vorotracing.py:536-543) */
int vt_permute_rows(const void *src, uint32_t rows, uint32_t row_bytes, const uint32_t *perm, void *dst,
                    vt_stream_t stream);

/*
 * Screen-tile lane permutation.  Replaces VoroTracingInfer._tile_perm
 * (vorotracing.py:606-625): perm (height*width) int32, lane t renders pixel
 * perm[t], tiles of tile_h x tile_w in row-major tile order (the reference
 * uses 4 x 8 for 32-wide warps; wave64 uses 8 x 8).
 */
int vt_tile_perm(uint32_t height, uint32_t width, uint32_t tile_h, uint32_t tile_w, int32_t *perm,
                 vt_stream_t stream);

/*
 * Launch order of the screen tiles of the tiled and camera inference
 * entries (an extension; the reference launches blocks in screen order).
 * tile_cost (u32, one per tile) is what such a call wrote to its tile_cost
 * argument: 18 x the longest walk's steps + the most face records searched by
 * one ray of the tile.  tile_order (u32, tiles + 1 words) receives the tiles
 * by decreasing cost bucket (8 buckets per octave of the cost over
 * [16, 2^20): floor(log2 c) and the next three bits of c; costs below 16 in
 * the last bucket, from 2^20 in the first), tiles of one bucket in screen
 * order, which keeps neighbouring tiles together; a call given it
 * launches tile tile_order[s] in slot s.  Launched longest first, a frame no
 * longer ends with a few long tiles running on an otherwise idle GPU.  Any
 * order gives bit-identical images (a ray's result does not depend on its
 * lane).
 * tile_order[tiles] receives the split count (ABI version 10): the number of
 * tiles whose cost exceeds 4/5 of sum(cost) / split_waves, 0 when
 * split_waves is 0.  split_waves is the number of waves the consuming launch
 * holds at once (below 2^24): a tile costing more than one such wave's mean
 * share still runs when the rest has drained.  The training backward runs
 * the first tile_order[tiles] tiles of its order as two half-waves each (pass
 * vt_train_bwd_resident_waves()), and so does the forward when the count is
 * non-zero (pass vt_train_fwd_resident_waves()); the inference entries
 * ignore the count (pass 0).
 * workspace: vt_tile_order_workspace_size(tiles) bytes, 8-byte aligned.
 */
size_t vt_tile_order_workspace_size(uint32_t tiles);
int vt_tile_order(const uint32_t *tile_cost, uint32_t tiles, uint32_t split_waves, uint32_t *tile_order,
                  void *workspace, vt_stream_t stream);
/* Waves of the training forward (24 per CU) and backward (16 per CU) that
 * the current device holds at once, the split_waves of their tile orders; 0
 * if the device query fails. */
uint32_t vt_train_fwd_resident_waves(void);
uint32_t vt_train_bwd_resident_waves(void);

/*
 * q8 quantisation.  Replaces VoroTracingInfer._quantize_to_uint8
 * (vorotracing.py:495-503): scale = fp32((vmax - vmin) / 255) (double
 * arithmetic), offset = vmin, q = clamp(rint((x - offset) * fp32(1/scale)),
 * 0, 255).  per_channel = 1 computes one (scale, offset) per RGB channel of
 * the texel-major map (cols % 3 == 0).  params out (device): 9 floats =
 * scale[3], offset[3], 1/scale[3] (all three equal when per-tensor).
 * workspace: vt_quantize_workspace_size() bytes.
 */
size_t vt_quantize_workspace_size(void);
int vt_quantize_u8(const float *x, uint32_t rows, uint32_t cols, int per_channel, uint8_t *q, float *params,
                   void *workspace, vt_stream_t stream);

/*
 * Backward epilogue of the training traversal, fused.  Replaces the
 * nan_to_num of the four gradients in TraceVoroTracing.backward
 * (_wrapper.py:189-198) and autograd's chain through the density activation
 * s = a * exp(raw) (vorotracing.py:346-347): in one pass,
 *   points/diffuse/specular gradients: NaN and +-inf -> 0, in place;
 *   density_grad_raw = (nan_to_num(density_grad_s) * a) * exp_raw
 *   (the operations and order of torch's MulBackward and ExpBackward).
 * exp_raw is exp(raw) as the forward computed it.  Counts are elements.
 */
int vt_grad_epilogue(float *points_grad, uint64_t points_n, float *diffuse_grad, uint64_t diffuse_n,
                     float *specular_grad, uint64_t specular_n, const float *density_grad_s, const float *exp_raw,
                     float activation_scale, uint32_t num_points, float *density_grad_raw, vt_stream_t stream);

/*
 * Optimizer step of the trainer, fused (trainer.py:233-265): the manual
 * regulariser gradients (specular: g += 2 w_s / numel * p; diffuse mean pull:
 * g += 2 w_d / numel * (p - mean over the cell's R*R texels, per channel)),
 * Adam (torch.optim.Adam: betas, eps, bias correction at `step`, counted from
 * 1; no weight decay) over the four parameter groups, then
 * density = min(density, density_max).  Parameters, gradients and the two
 * moment buffers of each group are f32 in the model's layouts (points
 * (N,3), density (N,1), diffuse (N, 3*Rd*Rd), specular (N, 3*Rs*Rs),
 * texel-major RGB).  lr: points, density, diffuse, specular (the trainer's
 * group order).  lr and betas are doubles: 1 - beta, the bias corrections and
 * lr / (1 - beta1^step) are formed in double and rounded once, as torch forms
 * them from Python floats.  Gradients are read, not written.  diff_res: 4, 8.
 */
int vt_adam_voro(float *points, float *points_grad, float *points_m, float *points_v, float *density,
                 float *density_grad, float *density_m, float *density_v, float *diffuse, float *diffuse_grad,
                 float *diffuse_m, float *diffuse_v, uint32_t diff_res, float *specular, float *specular_grad,
                 float *specular_m, float *specular_v, uint32_t spec_res, uint32_t num_points, const double lr[4],
                 double beta1, double beta2, float eps, uint32_t step, float specular_reg_weight,
                 float diffuse_mean_pull_weight, float density_max, vt_stream_t stream);

/*
 * Voronoi neighbours (the Delaunay adjacency) of a site set, built on the GPU.
 * Replaces the adjacency step of vorotracing.cuda.build_voronoi_adjacency
 * (cuda/__init__.py:16-46), which the reference delegates to Paragram.
 *   vt_voronoi_build: points (num_points, 3) f32 -> offsets u32
 *   (num_points+1) and *num_adjacency = offsets[num_points] (host).  Each
 *   cell is clipped in fp64 from a bounding box by the bisector planes of
 *   nearby sites; its neighbours are the sites whose planes keep a face, in
 *   ascending order (the set equals qhull's Delaunay neighbours for points in
 *   general position).  Synchronises `stream` (the host needs the total).
 *   Fails with VT_ERR_INVALID if a cell exceeds the per-cell capacity or a
 *   cut is degenerate (message gives the counts).
 *   vt_voronoi_adjacency: writes the lists into adjacency (num_adjacency
 *   entries; the caller adds any padding).
 *   workspace: vt_voronoi_workspace_size(num_points) bytes, the same buffer
 *   for both calls.
 */
size_t vt_voronoi_workspace_size(uint32_t num_points);
int vt_voronoi_build(const float *points, uint32_t num_points, uint32_t *offsets, uint32_t *num_adjacency,
                     void *workspace, vt_stream_t stream);
/*
 * vt_voronoi_build with a warm start: guess_offsets (num_points + 1) and
 * guess_adjacency (u32 CSR, e.g. the adjacency before the sites moved, as the
 * reference's training refresh can pass to Paragram: initial_guesses,
 * cuda/__init__.py:16-37) cut each cell first; the result is the same
 * neighbour sets as without guesses (out-of-range ids are ignored), found
 * faster when the guesses are close.  guess_adjacency holds num_guesses
 * entries (an argument since ABI version 7); a cell whose guess range runs
 * backwards or past them builds without guesses.  NULL, NULL, 0 =
 * vt_voronoi_build.
 */
int vt_voronoi_build_warm(const float *points, uint32_t num_points, const uint32_t *guess_offsets,
                          const uint32_t *guess_adjacency, uint32_t num_guesses, uint32_t *offsets,
                          uint32_t *num_adjacency, void *workspace, vt_stream_t stream);
int vt_voronoi_adjacency(uint32_t num_points, const uint32_t *offsets, uint32_t *adjacency, const void *workspace,
                         vt_stream_t stream);

/* fp16 Half4Texel padding.  Replaces VoroTracingInfer._pad_3to4 applied to
 * .half() maps (vorotracing.py:477-482, :505-512): f32 (rows, 3*T) ->
 * f16 (rows, 4*T), RNE cast, zero 4th channel. */
int vt_pad_3to4_f16(const float *x, uint32_t rows, uint32_t texels_per_row, uint16_t *out, vt_stream_t stream);

/*
 * Self-test of the device arithmetic shared by restatement with the CPU
 * checker (no reference counterpart): op 0 = exp, 1 = log, 2 = f32->f16 bits
 * (out as u16 in the low half of each u32), 3 = sin and 4 = cos of the camera
 * generator (arguments in [0, pi]), applied elementwise to n floats; op 5 =
 * the walk's exit-face order on n records (num, dp, bnum, bdp) of 4 floats
 * (dp, bdp > 0): out = 1 iff RN(num/dp) < RN(bnum/bdp) as the walk decides it;
 * op 6 = the walk's exit-face search on n rows of 26 floats (site, origin,
 * unit direction, face count <= 8 as u32 bits, 8 half4 face records as 16
 * u32; counts above 8 read as 8), out = 2 words per row: face index
 * (0xffffffff = none) and t1 bits; op 7 = the packed walk's search over one
 * chunk whose faces are reordered, on n rows of 30 floats (an op 6 row with
 * the records in slot order and zero records past the count, then the 8
 * slots' original indices as u16 in 4 words), out = the original index of
 * the exit face (0xffffffff = none) and t1 bits.
 */
int vt_math_probe(int op, const float *in, uint32_t *out, uint32_t n, vt_stream_t stream);

/*
 * Self-test of the half-precision atomic add of the f16-storage backward (no
 * reference counterpart; it stands in for the reference's atomicAdd on
 * __half, ray_integrator_octmap.cuh:1004-1007,1021-1024): thread i adds
 * values[i], rounded to half, to halves[index[i]] with the backward's own
 * atomic.  Indices at or past num_halves (even) are skipped.
 */
int vt_debug_f16_atomic_add(uint16_t *halves, uint32_t num_halves, const uint32_t *index, const float *values,
                            uint32_t n, vt_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif
