// vt_camera.h -- ray generation from a vt_camera (include/vt_abi.h), the
// step the reference performs in torch before each render
// (utils/__init__.py:85-130; datasets/datasets.py:126-136, :286-304).
// f32 with the library's arithmetic convention; the CPU checker restates it
// operation for operation.
#pragma once

#include "../../include/vt_abi.h"
#include "vt_device.h"

namespace vt {

// sin x and cos x for x in [0, pi]: reduced to [-pi/4, pi/4] against pi/2
// or pi, each held as hi + lo (hi - x is exact there by Sterbenz's lemma,
// so the reduced argument is rounded once), then the Taylor polynomials of
// degree 13 (sin) and 14 (cos) in Horner form in z = r^2 (truncation below
// 3e-14 on [-pi/4, pi/4]).
constexpr float PI_HI = 0x1.921fb6p+1f, PI_LO = -0x1.777a5cp-24f;
constexpr float PIO2_HI = 0x1.921fb6p+0f, PIO2_LO = -0x1.777a5cp-25f;
constexpr float PIO4 = 0.785398185f, PI3O4 = 2.35619450f;

__device__ __forceinline__ float sin_poly(float r)
{
    const float z = r * r;
    float p = 1.0f / 6227020800.0f;
    p = fma_(p, z, -1.0f / 39916800.0f);
    p = fma_(p, z, 1.0f / 362880.0f);
    p = fma_(p, z, -1.0f / 5040.0f);
    p = fma_(p, z, 1.0f / 120.0f);
    p = fma_(p, z, -1.0f / 6.0f);
    return fma_(r * z, p, r);
}

__device__ __forceinline__ float cos_poly(float r)
{
    const float z = r * r;
    float p = -1.0f / 87178291200.0f;
    p = fma_(p, z, 1.0f / 479001600.0f);
    p = fma_(p, z, -1.0f / 3628800.0f);
    p = fma_(p, z, 1.0f / 40320.0f);
    p = fma_(p, z, -1.0f / 720.0f);
    p = fma_(p, z, 1.0f / 24.0f);
    p = fma_(p, z, -0.5f);
    return fma_(z, p, 1.0f);
}

__device__ __forceinline__ float vt_sinf(float x)
{
    if (x <= PIO4)
        return sin_poly(x);
    if (x <= PI3O4)
        return cos_poly((PIO2_HI - x) + PIO2_LO); // sin x = cos(pi/2 - x)
    return sin_poly((PI_HI - x) + PI_LO);         // sin x = sin(pi - x)
}

__device__ __forceinline__ float vt_cosf(float x)
{
    if (x <= PIO4)
        return cos_poly(x);
    if (x <= PI3O4)
        return sin_poly((PIO2_HI - x) + PIO2_LO); // cos x = sin(pi/2 - x)
    return -cos_poly((PI_HI - x) + PI_LO);        // cos x = -cos(pi - x)
}

// Ray of pixel (u, v) of an H-row image: origin o, direction d (not yet
// normalised; the traversal normalises every ray it reads).
__device__ __forceinline__ void camera_ray(const vt_camera &c, uint32_t u, uint32_t v, uint32_t H, f3 &o, f3 &d)
{
    const float mx = ((float)u + c.pixel_offset - c.cx) / c.fx;
    const float my = ((float)v + c.pixel_offset - c.cy) / c.fy;
    f3 dc = mk(mx, my, 1.0f);
    if (c.model == VT_CAMERA_FISHEYE) {
        const float td = __builtin_sqrtf(fma_(my, my, mx * mx));
        dc = mk(0.0f, 0.0f, 1.0f);
        if (td > 0.0f) {
            // Newton on theta (1 + k1 theta^2 + k2 theta^4 + k3 theta^6 + k4 theta^8) = td
            float th = td;
            for (int it = 0; it < 12; ++it) {
                const float t2 = th * th;
                const float p = fma_(fma_(fma_(c.k[3], t2, c.k[2]), t2, c.k[1]), t2, c.k[0]);
                const float q =
                    fma_(fma_(fma_(9.0f * c.k[3], t2, 7.0f * c.k[2]), t2, 5.0f * c.k[1]), t2, 3.0f * c.k[0]);
                const float g = fma_(th * t2, p, th) - td;
                const float dg = fma_(t2, q, 1.0f);
                th = th - g / dg;
            }
            th = __builtin_fminf(__builtin_fmaxf(th, 0.0f), PI_HI);
            const float s = vt_sinf(th) / td;
            dc = mk(mx * s, my * s, vt_cosf(th));
        }
    }
    dc = divs(dc, __builtin_sqrtf(dot(dc, dc)));
    d = mk(dot(mk(c.R[0], c.R[1], c.R[2]), dc), dot(mk(c.R[3], c.R[4], c.R[5]), dc),
           dot(mk(c.R[6], c.R[7], c.R[8]), dc));
    const float sv = H > 1 ? (float)v / (float)(H - 1) : 0.0f;
    o = mk(fma_(sv, c.rolling[0], c.t[0]), fma_(sv, c.rolling[1], c.t[1]), fma_(sv, c.rolling[2], c.t[2]));
}


} // namespace vt
