// vt_prims.h -- device primitives shared by the preparation kernels:
// exclusive scan, stable LSD radix sort of (key, value) pairs, bounding box.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace vt {

// Words of scratch (u32) needed by exclusive_scan_u32 for n elements.
size_t scan_workspace_words(uint32_t n);
// out[i] = sum(in[0..i)), u32 wrap-around; in == out allowed.
int exclusive_scan_u32(const uint32_t *in, uint32_t *out, uint32_t n, uint32_t *ws, hipStream_t s);

// Words of scratch (u32) needed by radix_sort_pass for n elements.
size_t radix_pass_workspace_words(uint32_t n);
// One stable counting-sort pass on the 8-bit digit (key >> shift) & 255:
// (kin, vin)[0..n) scattered to (kout, vout) in ascending digit order, equal
// digits in input order.  Outputs must not alias the inputs.
int radix_sort_pass(const uint32_t *kin, const uint32_t *vin, uint32_t *kout, uint32_t *vout, uint32_t n, int shift,
                    uint32_t *ws, hipStream_t s);

// Words of scratch (u32) needed by radix_sort_pairs for n elements.
size_t radix_sort_workspace_words(uint32_t n);
// Stable ascending sort of keys[0..n) (the low `bits` bits are compared),
// values permuted alongside.  Results are left in keys / vals.
int radix_sort_pairs(uint32_t *keys, uint32_t *vals, uint32_t n, int bits, uint32_t *ws, hipStream_t s);

// Per-axis min / max of (n, 3) f32 points into bbox6 = {min xyz, max xyz}
// (device).  ws: 6 words of scratch.
int bbox3(const float *points, uint32_t n, float *bbox6, uint32_t *ws, hipStream_t s);

// Ordered-integer encoding of floats (monotone in the float order) used for
// min / max reductions with integer atomics.
__device__ __forceinline__ int32_t f2ord(float f)
{
    int32_t b = __builtin_bit_cast(int32_t, f);
    return b >= 0 ? b : (b ^ 0x7fffffff);
}
__device__ __forceinline__ float ord2f(int32_t o)
{
    int32_t b = o >= 0 ? o : (o ^ 0x7fffffff);
    return __builtin_bit_cast(float, b);
}

} // namespace vt
