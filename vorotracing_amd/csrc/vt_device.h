// vt_device.h -- device arithmetic and record access shared by the
// traversal kernels (gfx950, wave64).
//
// Arithmetic convention (identical, by restatement, to the CPU checker):
//   dot(a, b) = fma(a2, b2, fma(a1, b1, a0 * b0));
//   every "a * b + c" the reference writes is an explicit fma; nothing else is
//   contracted (the library is compiled with -ffp-contract=off);
//   division and sqrt are IEEE correctly rounded
//   (-fhip-fp32-correctly-rounded-divide-sqrt);
//   exp/log are vt_expf/vt_logf below; f32->f16 is v_cvt_f16_f32 (RNE).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/vt_abi.h"

namespace vt {

constexpr uint32_t NONE = 0xffffffffu;

struct f3 {
    float x, y, z;
};

__device__ __forceinline__ f3 mk(float x, float y, float z) { return f3{x, y, z}; }
__device__ __forceinline__ f3 sub(f3 a, f3 b) { return mk(a.x - b.x, a.y - b.y, a.z - b.z); }
__device__ __forceinline__ f3 add(f3 a, f3 b) { return mk(a.x + b.x, a.y + b.y, a.z + b.z); }
__device__ __forceinline__ f3 divs(f3 a, float s) { return mk(a.x / s, a.y / s, a.z / s); }
__device__ __forceinline__ float fma_(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ float dot(f3 a, f3 b) { return fma_(a.z, b.z, fma_(a.y, b.y, a.x * b.x)); }
// acc + s * a, contracted
__device__ __forceinline__ f3 vfma(float s, f3 a, f3 acc)
{
    return mk(fma_(s, a.x, acc.x), fma_(s, a.y, acc.y), fma_(s, a.z, acc.z));
}

__device__ __forceinline__ float bits_f(uint32_t b) { return __builtin_bit_cast(float, b); }
__device__ __forceinline__ uint32_t f_bits(float f) { return __builtin_bit_cast(uint32_t, f); }

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// exp(x): Cody & Waite two-constant reduction x = k ln2 + r (|r| <= ln2/2),
// degree-7 Taylor polynomial of e^r, scaling by 2^k with one final rounding.
// ln2 = LN2_HI (ln2 rounded to 16 fractional bits, k*LN2_HI exact) + LN2_LO.
__device__ __forceinline__ float vt_expf(float x)
{
    if (x != x)
        return x;
    if (x > 88.72283935546875f)
        return __builtin_huge_valf();
    if (x < -103.972084045410156f)
        return 0.0f;
    float kf = __builtin_rintf(x * 1.44269502162933349609375f);
    float r = fma_(kf, -0.693145751953125f, x);
    r = fma_(kf, -1.42860676533018704e-06f, r);
    float q = 1.0f / 5040.0f;
    q = fma_(q, r, 1.0f / 720.0f);
    q = fma_(q, r, 1.0f / 120.0f);
    q = fma_(q, r, 1.0f / 24.0f);
    q = fma_(q, r, 1.0f / 6.0f);
    q = fma_(q, r, 0.5f);
    float e = fma_(q, r * r, r) + 1.0f;
    int k = (int)kf;
    if (k > 127)
        return (e * bits_f(0x7f000000u)) * bits_f((uint32_t)k << 23);
    if (k < -126)
        return (e * bits_f((uint32_t)(k + 191) << 23)) * bits_f(63u << 23);
    return e * bits_f((uint32_t)(k + 127) << 23);
}

// log(x): x = 2^e m, m in [sqrt(1/2), sqrt(2)), s = (m-1)/(m+1),
// log m = 2 atanh(s) = 2s + 2s^3/3 + ... + 2s^11/11, plus e ln2 (split above).
__device__ __forceinline__ float vt_logf(float x)
{
    if (x != x || x < 0.0f)
        return __builtin_nanf("");
    if (x == 0.0f)
        return -__builtin_huge_valf();
    if (x == __builtin_huge_valf())
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
    p = fma_(p, z, 2.0f / 9.0f);
    p = fma_(p, z, 2.0f / 7.0f);
    p = fma_(p, z, 2.0f / 5.0f);
    p = fma_(p, z, 2.0f / 3.0f);
    float lm = fma_(s * z, p, 2.0f * s);
    float ef = (float)e;
    return fma_(ef, 0.693145751953125f, fma_(ef, 1.42860676533018704e-06f, lm));
}

__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + vt_expf(-x)); }

// LDS writes of some lanes of a wave visible to the wave's other lanes (and
// not reordered by the compiler across the point).
__device__ __forceinline__ void wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// Largest x over the 64 lanes of the wave (every lane must be active).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x)
{
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1)
        x = max(x, (uint32_t)__shfl_xor((int)x, k));
    return x;
}

// Number of set bits of m below the calling lane.
__device__ __forceinline__ uint32_t lane_rank(uint64_t m)
{
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Blocks are dispatched round-robin over the 8 XCDs of an MI355X, each with
// its own L2.  Remap so that each XCD runs one contiguous range of logical
// blocks (neighbouring rays -> neighbouring cells -> same L2).
__device__ __forceinline__ uint32_t xcd_block()
{
    uint32_t G = gridDim.x, b = blockIdx.x;
    uint32_t xcd = b & 7u, local = b >> 3;
    uint32_t q = G >> 3, r = G & 7u;
    return xcd < r ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
}

__device__ __forceinline__ uint32_t xcd_block_linear() { return xcd_block() * blockDim.x + threadIdx.x; }

// Blocks dealt to the 8 XCDs in chunks of C consecutive logical blocks,
// round-robin: each XCD still sees runs of C neighbouring blocks (neighbouring
// screen tiles share cells in its L2), but every XCD gets a share of every
// screen region, so that one XCD does not end up with all the expensive
// tiles of a frame.  Blocks past the last full round of 8 C keep their index.
template <uint32_t C> __device__ __forceinline__ uint32_t xcd_interleaved_block()
{
    constexpr uint32_t S = 8 * C;
    const uint32_t b = blockIdx.x, full = gridDim.x / S * S;
    if (b >= full)
        return b;
    const uint32_t local = b >> 3;
    return (local / C) * S + (b & 7u) * C + local % C;
}

// ---------------------------------------------------------------------------
// octahedral map (ray_integrator_octmap.cuh:17-55)

template <int R> __device__ __forceinline__ void oct_encode(f3 d, float &tu, float &tv)
{
    float l1 = (__builtin_fabsf(d.x) + __builtin_fabsf(d.y)) + __builtin_fabsf(d.z);
    float inv = 1.0f / __builtin_fmaxf(l1, 1e-10f);
    float u = d.x * inv;
    float v = d.y * inv;
    if (d.z < 0.0f) {
        float ou = (1.0f - __builtin_fabsf(v)) * __builtin_copysignf(1.0f, u);
        float ov = (1.0f - __builtin_fabsf(u)) * __builtin_copysignf(1.0f, v);
        u = ou;
        v = ov;
    }
    tu = fma_(fma_(u, 0.5f, 0.5f), (float)R, -0.5f);
    tv = fma_(fma_(v, 0.5f, 0.5f), (float)R, -0.5f);
}

struct Bilinear {
    int i00, i10, i01, i11;
    float w00, w10, w01, w11;
};

// oct_wrap_index (ray_integrator_octmap.cuh:36-55) restricted to texel
// coordinates in [-1, R] (R a power of two),
// the only ones a bilinear tap of an encoded direction reaches: oct_encode
// gives |u|, |v| <= 1 (|x| <= l1 after rounding, and x * RN(1/l1) rounds to
// at most 1), so tex_u lies in [-0.5, R - 0.5], floor(tex_u) in [-1, R - 1]
// and floor(tex_u) + 1 in [0, R].  There the general form reduces to
// wrap = u mod R and one fold for each coordinate outside [0, R).
template <int R> __device__ __forceinline__ int oct_wrap_edge(int u, int v)
{
    static_assert((R & (R - 1)) == 0, "R must be a power of two");
    int wu = u & (R - 1);
    int wv = v & (R - 1);
    bool fu = (unsigned)u >= (unsigned)R;
    bool fv = (unsigned)v >= (unsigned)R;
    if (fu != fv) {
        wu = R - 1 - wu;
        wv = R - 1 - wv;
    }
    return wv * R + wu;
}

template <int R> __device__ __forceinline__ Bilinear bilinear_setup(float u, float v)
{
    Bilinear b;
    int u0 = (int)__builtin_floorf(u);
    int v0 = (int)__builtin_floorf(v);
    float fu = u - (float)u0;
    float fv = v - (float)v0;
    b.i00 = oct_wrap_edge<R>(u0, v0);
    b.i10 = oct_wrap_edge<R>(u0 + 1, v0);
    b.i01 = oct_wrap_edge<R>(u0, v0 + 1);
    b.i11 = oct_wrap_edge<R>(u0 + 1, v0 + 1);
    b.w00 = (1.0f - fu) * (1.0f - fv);
    b.w10 = fu * (1.0f - fv);
    b.w01 = (1.0f - fu) * fv;
    b.w11 = fu * fv;
    return b;
}

// The bilinear tap of (u, v) as an entry of a footprint table (vt_quad_maps:
// entry (ex, ey), 0 <= ex, ey <= R, holds the four wrapped texels of the
// taps with floor coordinates (ex - 1, ey - 1)): q = (v0 + 1) (R + 1) + u0 + 1
// and the weights of bilinear_setup.  u0, v0 lie in [-1, R - 1] for every
// encoded direction (see oct_wrap_edge; a NaN converts to 0); the clamp keeps
// any other input inside the table.
template <int R> __device__ __forceinline__ Bilinear bilinear_quad(float u, float v)
{
    Bilinear b;
    int u0 = (int)__builtin_floorf(u);
    int v0 = (int)__builtin_floorf(v);
    float fu = u - (float)u0;
    float fv = v - (float)v0;
    const int cu = u0 < -1 ? -1 : (u0 > R - 1 ? R - 1 : u0);
    const int cv = v0 < -1 ? -1 : (v0 > R - 1 ? R - 1 : v0);
    b.i00 = (cv + 1) * (R + 1) + cu + 1;
    b.i10 = b.i01 = b.i11 = 0;
    b.w00 = (1.0f - fu) * (1.0f - fv);
    b.w10 = fu * (1.0f - fv);
    b.w01 = (1.0f - fu) * fv;
    b.w11 = fu * fv;
    return b;
}

// w00*a + w10*b + w01*c + w11*d, left to right, contracted
__device__ __forceinline__ float bil_mix(const Bilinear &b, float a, float bb, float c, float d)
{
    return fma_(b.w11, d, fma_(b.w01, c, fma_(b.w10, bb, b.w00 * a)));
}

// direction of the diffuse probe: normalize(o + t0 d - site), or d
// sqrtf(x) > 1e-8f exactly when x > PROBE_LEN2_MIN (sqrt is correctly rounded
// and monotone; the constant is the largest float whose root rounds to at
// most 1e-8f), so probe_dir's length test needs no square root.
constexpr float PROBE_LEN2_MIN = 0x1.cd2b2ap-54f;

__device__ __forceinline__ f3 probe_dir(f3 o, f3 d, float t0, f3 site)
{
    f3 hit = mk(fma_(t0, d.x, o.x), fma_(t0, d.y, o.y), fma_(t0, d.z, o.z));
    f3 dv = sub(hit, site);
    float len = __builtin_sqrtf(dot(dv, dv));
    if (len > 1e-8f)
        return divs(dv, len);
    return d;
}

// ---------------------------------------------------------------------------
// loads

__device__ __forceinline__ f3 load_site(const float *p, uint32_t i)
{
    const float *q = p + 3 * (size_t)i;
    return mk(q[0], q[1], q[2]);
}

// Ray (camera.h:5-8) with the kernel's re-normalisation d /= |d|
// (tracing_octmap.cu:180, :577)
__device__ __forceinline__ void load_ray(const float *rays, uint32_t r, f3 &o, f3 &d)
{
    const float *q = rays + 6 * (size_t)r;
    o = mk(q[0], q[1], q[2]);
    f3 dd = mk(q[3], q[4], q[5]);
    float nrm = __builtin_sqrtf(dot(dd, dd));
    d = divs(dd, nrm);
}

// face record (half4 offset) -> f32 offset
__device__ __forceinline__ f3 load_face(const uint2 *adj_diff, uint32_t e)
{
    uint2 w = adj_diff[e];
    return mk(h2f((uint16_t)(w.x & 0xffffu)), h2f((uint16_t)(w.x >> 16)), h2f((uint16_t)(w.y & 0xffffu)));
}

// per-ray walk statistics (the vt_ray_stats record)
struct Stats {
    uint32_t n, visits, faces, exits, integrated, shaded;
    uint64_t hash;
};

constexpr uint32_t STATS_WORDS = sizeof(vt_ray_stats) / 4;
static_assert(sizeof(vt_ray_stats) == 4 * (8 + VT_STATS_LOG), "vt_ray_stats is 8 counter words and the log");

template <bool ON> struct StatsAcc {
    // visit() takes a cell's face count, or any cost-like count when false
    static constexpr bool EXACT_FACES = false;
    uint32_t faces = 0; // face records searched (a launch-order cost; dropped when unread)
    __device__ __forceinline__ void begin(void *, uint32_t) {}
    __device__ __forceinline__ void visit(uint32_t, uint32_t nf) { faces += nf; }
    __device__ __forceinline__ uint32_t face_count() const { return faces; }
    __device__ __forceinline__ void exit() {}
    __device__ __forceinline__ void integrate() {}
    __device__ __forceinline__ void shade() {}
    __device__ __forceinline__ void store(void *, uint32_t, uint32_t) {}
};

template <> struct StatsAcc<true> {
    static constexpr bool EXACT_FACES = true;
    Stats s{0, 0, 0, 0, 0, 0, 1469598103934665603ull};
    uint32_t *log = nullptr; // first_cells of this ray's record
    // the record of ray r (NONE: no record)
    __device__ __forceinline__ void begin(void *out, uint32_t r)
    {
        if (out && r != NONE)
            log = (uint32_t *)out + STATS_WORDS * (size_t)r + 8;
    }
    __device__ __forceinline__ void visit(uint32_t cell, uint32_t nf)
    {
        if (log && s.visits < VT_STATS_LOG)
            log[s.visits] = cell;
        s.visits++;
        s.faces += nf;
        s.hash = (s.hash ^ (uint64_t)cell) * 1099511628211ull;
    }
    __device__ __forceinline__ uint32_t face_count() const { return s.faces; }
    __device__ __forceinline__ void exit() { s.exits++; }
    __device__ __forceinline__ void integrate() { s.integrated++; }
    __device__ __forceinline__ void shade() { s.shaded++; }
    __device__ __forceinline__ void store(void *out, uint32_t r, uint32_t n)
    {
        uint32_t *o = (uint32_t *)out + STATS_WORDS * (size_t)r;
        for (uint32_t k = s.visits; k < VT_STATS_LOG; ++k)
            o[8 + k] = NONE;
        o[0] = n;
        o[1] = s.visits;
        o[2] = s.faces;
        o[3] = s.exits;
        o[4] = s.integrated;
        o[5] = s.shaded;
        o[6] = (uint32_t)(s.hash & 0xffffffffu);
        o[7] = (uint32_t)(s.hash >> 32);
    }
};

} // namespace vt
