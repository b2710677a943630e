// vt_optim.hip -- the element-wise work around the training backward, fused:
//   * the backward epilogue of TraceVoroTracing (_wrapper.py:189-198:
//     nan_to_num of the four gradients) with the density activation chain
//     s = a exp(raw) (vorotracing.py:346-347) that autograd would run next;
//   * the optimizer step of the trainer (trainer.py:233-265): the manual
//     specular and diffuse-mean-pull regulariser gradients, Adam
//     (torch.optim.Adam, eps 1e-15, no weight decay) over the four parameter
//     groups, and the log-density clamp.
// One launch each instead of the ~15 element-wise passes torch runs.
#include "vt_internal.h"

#include <cmath>

namespace vt {

constexpr int OPT_BLOCK = 256;

__device__ __forceinline__ float nan_to_zero(float x)
{
    // torch.nan_to_num(x, nan=0, posinf=0, neginf=0)
    return (x - x == 0.0f) ? x : 0.0f;
}

constexpr int EPI_PER_THREAD = 4;
constexpr int EPI_CHUNK = OPT_BLOCK * EPI_PER_THREAD; // elements per block

struct EpilogueArgs {
    float *g[3];     // points, diffuse, specular gradients (cleaned in place)
    uint64_t n[4];   // their element counts, then the density's
    uint32_t blocks[4];
    const float *gs; // gradient w.r.t. the activated density s
    const float *e;  // exp(raw), as saved by the forward
    float a;         // activation scale
    float *graw;     // gradient w.r.t. the raw log-density
};

// Blocks in ranges per tensor [points | diffuse | specular | density], each
// block a chunk of EPI_CHUNK elements, lanes striding by the block size.
__global__ __launch_bounds__(OPT_BLOCK) void grad_epilogue_kernel(EpilogueArgs a)
{
    uint32_t b = blockIdx.x;
    int t = 0;
    while (t < 3 && b >= a.blocks[t]) {
        b -= a.blocks[t];
        ++t;
    }
    const uint64_t k0 = (uint64_t)b * EPI_CHUNK + threadIdx.x, n = a.n[t];
    if (t < 3) {
        float *g = a.g[t];
#pragma unroll
        for (int r = 0; r < EPI_PER_THREAD; ++r) {
            const uint64_t k = k0 + (uint64_t)r * OPT_BLOCK;
            if (k < n)
                g[k] = nan_to_zero(g[k]);
        }
    } else {
#pragma unroll
        for (int r = 0; r < EPI_PER_THREAD; ++r) {
            const uint64_t k = k0 + (uint64_t)r * OPT_BLOCK;
            if (k < n) // autograd of s = a * exp(raw): MulBackward (g * a), then ExpBackward (* exp(raw))
                a.graw[k] = (nan_to_zero(a.gs[k]) * a.a) * a.e[k];
        }
    }
}

struct AdamGroup {
    float *p, *g, *m, *v;
    uint64_t n;
    float step_size; // lr / (1 - beta1^t), formed in double like torch's Python scalars
};

struct AdamArgs {
    AdamGroup grp[4]; // points, density, specular, diffuse
    float beta1, beta2, eps;
    float omb1, omb2;       // 1 - beta1, 1 - beta2 (rounded from double, as torch's Python scalars)
    float bc2_sqrt;         // sqrt(1 - beta2^t)
    float spec_scale;       // 2 w_spec / numel(specular), 0 when off
    float diff_scale;       // 2 w_pull / numel(diffuse), 0 when off
    float density_max;      // clamp of the log-density after the step
    uint32_t diff_texels;   // R^2 texels (3 channels each) per diffuse cell
    uint32_t blocks[4];     // blocks of each group, in order
};

// One Adam update of parameter p with gradient g.
__device__ __forceinline__ void adam_update(float &p, float &m, float &v, float g, const AdamArgs &a, float step_size)
{
    m = a.beta1 * m + a.omb1 * g;
    v = a.beta2 * v + a.omb2 * (g * g);
    const float denom = __builtin_sqrtf(v) / a.bc2_sqrt + a.eps;
    p = p - step_size * (m / denom);
}

// Blocks [0, b0) points, [b0, b0+b1) density, then specular, then diffuse.
// Diffuse: a group of R^2 lanes per cell (one texel, 3 channels each), the
// per-cell channel means reduced over the group.
template <int TEX>
__global__ __launch_bounds__(OPT_BLOCK) void adam_voro_kernel(AdamArgs a)
{
    uint32_t b = blockIdx.x;
    int t = 0;
    while (t < 3 && b >= a.blocks[t]) {
        b -= a.blocks[t];
        ++t;
    }
    const AdamGroup &G = a.grp[t];
    if (t < 3) {
        const uint64_t i = (uint64_t)b * OPT_BLOCK + threadIdx.x;
        if (i >= G.n)
            return;
        float g = G.g[i], p = G.p[i], m = G.m[i], v = G.v[i];
        if (t == 2)
            g = g + a.spec_scale * p; // spec.grad.add_(spec, alpha=scale)
        adam_update(p, m, v, g, a, G.step_size);
        if (t == 1)
            p = __builtin_fminf(p, a.density_max); // density.clamp_(max=...)
        G.p[i] = p;
        G.m[i] = m;
        G.v[i] = v;
        return;
    }
    // diffuse: TEX lanes per cell, cells_per_block = OPT_BLOCK / TEX
    const uint64_t cell = (uint64_t)b * (OPT_BLOCK / TEX) + threadIdx.x / TEX;
    const uint64_t cells = G.n / (3ull * TEX);
    const bool live = cell < cells;
    const uint64_t base = (cell * TEX + threadIdx.x % TEX) * 3;
    float p[3] = {0.0f, 0.0f, 0.0f}, s[3];
    if (live)
        for (int c = 0; c < 3; ++c)
            p[c] = G.p[base + c];
    for (int c = 0; c < 3; ++c) {
        s[c] = p[c];
        for (int o = 1; o < TEX; o <<= 1) // sum over the cell's TEX lanes
            s[c] += __shfl_xor(s[c], o, TEX);
    }
    if (!live)
        return;
    for (int c = 0; c < 3; ++c) {
        const float mean = s[c] / (float)TEX;
        float g = G.g[base + c];
        g = g + a.diff_scale * p[c]; // grad.add_(diff, alpha=scale)
        g = g + (-a.diff_scale) * mean; // grad.add_(mean, alpha=-scale)
        float pc = p[c], m = G.m[base + c], v = G.v[base + c];
        adam_update(pc, m, v, g, a, G.step_size);
        G.p[base + c] = pc;
        G.m[base + c] = m;
        G.v[base + c] = v;
    }
}

} // namespace vt

using namespace vt;

extern "C" int vt_grad_epilogue(float *points_grad, uint64_t points_n, float *diffuse_grad, uint64_t diffuse_n,
                                float *specular_grad, uint64_t specular_n, const float *density_grad_s,
                                const float *exp_raw, float activation_scale, uint32_t num_points,
                                float *density_grad_raw, vt_stream_t stream)
{
    clear_error();
    VT_REQUIRE((points_grad || !points_n) && (diffuse_grad || !diffuse_n) && (specular_grad || !specular_n) &&
                   ((density_grad_s && exp_raw && density_grad_raw) || !num_points),
               "null pointer argument");
    EpilogueArgs a{};
    a.g[0] = points_grad;
    a.g[1] = diffuse_grad;
    a.g[2] = specular_grad;
    a.n[0] = points_n;
    a.n[1] = diffuse_n;
    a.n[2] = specular_n;
    a.n[3] = num_points;
    a.gs = density_grad_s;
    a.e = exp_raw;
    a.a = activation_scale;
    a.graw = density_grad_raw;
    uint64_t blocks = 0;
    for (int t = 0; t < 4; ++t) {
        a.blocks[t] = (uint32_t)((a.n[t] + EPI_CHUNK - 1) / EPI_CHUNK);
        blocks += a.blocks[t];
    }
    if (blocks == 0)
        return VT_OK;
    VT_REQUIRE(blocks < (1ull << 31), "too many elements");
    grad_epilogue_kernel<<<(uint32_t)blocks, OPT_BLOCK, 0, as_stream(stream)>>>(a);
    VT_LAUNCH_CHECK("grad_epilogue_kernel");
    return VT_OK;
}

extern "C" int vt_adam_voro(float *points, float *points_grad, float *points_m, float *points_v, float *density,
                            float *density_grad, float *density_m, float *density_v, float *diffuse,
                            float *diffuse_grad, float *diffuse_m, float *diffuse_v, uint32_t diff_res,
                            float *specular, float *specular_grad, float *specular_m, float *specular_v,
                            uint32_t spec_res, uint32_t num_points, const double lr[4], double beta1, double beta2,
                            float eps, uint32_t step, float specular_reg_weight, float diffuse_mean_pull_weight,
                            float density_max, vt_stream_t stream)
{
    clear_error();
    if (num_points == 0)
        return VT_OK;
    VT_REQUIRE(points && points_grad && points_m && points_v && density && density_grad && density_m && density_v &&
                   diffuse && diffuse_grad && diffuse_m && diffuse_v && specular && specular_grad && specular_m &&
                   specular_v && lr,
               "null pointer argument");
    VT_REQUIRE(step >= 1, "step counts from 1, got %u", step);
    VT_REQUIRE(diff_res == 4 || diff_res == 8, "diffuse resolution %u not compiled (4, 8)", diff_res);
    VT_REQUIRE(spec_res >= 1, "specular resolution must be positive");
    AdamArgs a{};
    const uint64_t n = num_points;
    const uint64_t sizes[4] = {3 * n, n, 3ull * spec_res * spec_res * n, 3ull * diff_res * diff_res * n};
    float *P[4] = {points, density, specular, diffuse}, *Gr[4] = {points_grad, density_grad, specular_grad, diffuse_grad};
    float *M[4] = {points_m, density_m, specular_m, diffuse_m}, *V[4] = {points_v, density_v, specular_v, diffuse_v};
    // lr order of the caller: points, density, diffuse, specular (trainer.py:505-524)
    const double L[4] = {lr[0], lr[1], lr[3], lr[2]};
    const double bc1 = 1.0 - std::pow(beta1, (double)step);
    uint64_t nblocks = 0;
    for (int t = 0; t < 4; ++t) {
        a.grp[t] = AdamGroup{P[t], Gr[t], M[t], V[t], sizes[t], (float)(L[t] / bc1)};
        const uint64_t per = t < 3 ? OPT_BLOCK : (uint64_t)OPT_BLOCK / (diff_res * diff_res) * 3 * diff_res * diff_res;
        a.blocks[t] = (uint32_t)((sizes[t] + per - 1) / per);
        nblocks += a.blocks[t];
    }
    VT_REQUIRE(nblocks < (1ull << 31), "too many elements");
    a.beta1 = (float)beta1;
    a.beta2 = (float)beta2;
    a.eps = eps;
    a.omb1 = (float)(1.0 - beta1);
    a.omb2 = (float)(1.0 - beta2);
    a.bc2_sqrt = (float)std::sqrt(1.0 - std::pow(beta2, (double)step));
    a.spec_scale = specular_reg_weight > 0.0f ? (float)(2.0 * specular_reg_weight / (double)sizes[2]) : 0.0f;
    a.diff_scale = diffuse_mean_pull_weight > 0.0f ? (float)(2.0 * diffuse_mean_pull_weight / (double)sizes[3]) : 0.0f;
    a.density_max = density_max;
    a.diff_texels = diff_res * diff_res;
    if (diff_res == 4)
        adam_voro_kernel<16><<<(uint32_t)nblocks, OPT_BLOCK, 0, as_stream(stream)>>>(a);
    else
        adam_voro_kernel<64><<<(uint32_t)nblocks, OPT_BLOCK, 0, as_stream(stream)>>>(a);
    VT_LAUNCH_CHECK("adam_voro_kernel");
    return VT_OK;
}
