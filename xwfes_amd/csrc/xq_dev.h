// xq_dev.h -- the activation operand of the int8-MFMA row-dot GEMV (k_mfma.hip):
// its buffer layout and the wave-level routine that quantises one
// 256-element block of one activation row into it.
//
// Layout for a contraction of K (a multiple of 256), activation rows m < 8:
//   frag   K * 16 B   two int8 limbs per element in MFMA A-operand order
//   xs32   K B        32-element limb sums, 6-bit lo / signed hi split
//   xs16   2K B       16-element limb sums, same split
//   scale  K / 32 f   block scale s[sb][m] = max|x_block| / 127
//   ssq    K / 32 f   per-block sums of x^2 (RMS-normed inputs only)
// x ~= s * (a + b / 256) with |a|, |b| <= 127.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

struct XqPtrs {
    int8_t* frag;
    int8_t* xs32;
    int8_t* xs16;
    float* scale;
    float* ssq;
};

__host__ __device__ inline XqPtrs xq_ptrs(int8_t* xq, int64_t K) {
    XqPtrs p;
    p.frag = xq;
    p.xs32 = xq + K * 16;
    p.xs16 = p.xs32 + K;
    p.scale = (float*)(p.xs16 + 2 * K);
    p.ssq = p.scale + K / 32;
    return p;
}

// One wave writes block sb of row m: lane l holds elements 4l .. 4l+3 in v
// (zeros for rows past the live ones).
__device__ __forceinline__ void xq_emit(const float* v, int64_t sb, int m, int l, const XqPtrs& o) {
#pragma clang fp contract(off)
    float mx = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) mx = fmaxf(mx, __shfl_xor(mx, s, 64));
    const float q = mx > 0.f ? 127.f / mx : 0.f;
    if (l == 0) o.scale[sb * 8 + m] = mx > 0.f ? mx / 127.f : 0.f;
    int sa = 0, sbb = 0;
    uint32_t pa = 0, pb = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const float y = v[t] * q;
        const float a = rintf(y);
        float bf = rintf((y - a) * 256.f);
        bf = fminf(fmaxf(bf, -127.f), 127.f);
        const int ai = (int)a, bi = (int)bf;
        sa += ai;
        sbb += bi;
        pa |= (uint32_t)(ai & 0xFF) << (8 * t);
        pb |= (uint32_t)(bi & 0xFF) << (8 * t);
    }
    // fragment bytes: element 4l+t of the super-block sits in 32-block
    // kb = 8 sb + l/8, half (l%8)/4, byte 4(l%4) + t
    const int64_t kb = sb * 8 + (l >> 3);
    const int half = (l & 7) >> 2, byte = 4 * (l & 3);
    *(uint32_t*)(o.frag + ((kb * 2 + half) * 16 + m) * 16 + byte) = pa;
    *(uint32_t*)(o.frag + ((kb * 2 + half) * 16 + 8 + m) * 16 + byte) = pb;
    // 16-element sums (4 lanes), split into 6-bit lo / signed hi
#pragma unroll
    for (int s = 1; s < 4; s <<= 1) {
        sa += __shfl_xor(sa, s, 64);
        sbb += __shfl_xor(sbb, s, 64);
    }
    if ((l & 3) == 0) {
        const int s16 = l >> 2;
        o.xs16[(sb * 32 + m) * 16 + s16] = (int8_t)(sa & 63);
        o.xs16[(sb * 32 + 16 + m) * 16 + s16] = (int8_t)(sa >> 6);
        o.xs16[(sb * 32 + 8 + m) * 16 + s16] = (int8_t)(sbb & 63);
        o.xs16[(sb * 32 + 24 + m) * 16 + s16] = (int8_t)(sbb >> 6);
    }
    // 32-element sums (8 lanes)
    sa += __shfl_xor(sa, 4, 64);
    sbb += __shfl_xor(sbb, 4, 64);
    if ((l & 7) == 0) {
        const int j = l >> 3;
        o.xs32[(sb * 32 + m) * 8 + j] = (int8_t)(sa & 63);
        o.xs32[(sb * 32 + 16 + m) * 8 + j] = (int8_t)(sa >> 6);
        o.xs32[(sb * 32 + 8 + m) * 8 + j] = (int8_t)(sbb & 63);
        o.xs32[(sb * 32 + 24 + m) * 8 + j] = (int8_t)(sbb >> 6);
    }
}

// The same operand in the layout of the v_mfma_i32_16x16x32_i8 row-dot GEMV
// (k_rowdot.hip), where the activations are the A operand (16 rows = limb a
// of rows m = 0..7, then limb b) and the weights the B operand.  Same sizes
// and the same scale / ssq arrays as above; per super-block sb:
//   frag   [sb][lane 64][64 B]  lane L = 16 g + r (A row r), byte 8 j + e =
//                               element 32 j + 8 g + e (sub-block j)
//   xs32   [sb][row 16][16 B]   32-element limb sums: bytes j = lo 6 bits,
//                               8 + j = signed hi (sum >> 6)
//   xs16   [sb][row 16][32 B]   16-element limb sums: bytes s / 16 + s
// One wave writes block sb of row m: lane l holds elements 4l .. 4l+3 in v
// (zeros for rows past the live ones).
__device__ __forceinline__ void xq16_emit(const float* v, int64_t sb, int m, int l, const XqPtrs& o) {
#pragma clang fp contract(off)
    float mx = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) mx = fmaxf(mx, __shfl_xor(mx, s, 64));
    const float q = mx > 0.f ? 127.f / mx : 0.f;
    if (l == 0) o.scale[sb * 8 + m] = mx > 0.f ? mx / 127.f : 0.f;
    int sa = 0, sbb = 0;
    uint32_t pa = 0, pb = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const float y = v[t] * q;
        const float a = rintf(y);
        float bf = rintf((y - a) * 256.f);
        bf = fminf(fmaxf(bf, -127.f), 127.f);
        const int ai = (int)a, bi = (int)bf;
        sa += ai;
        sbb += bi;
        pa |= (uint32_t)(ai & 0xFF) << (8 * t);
        pb |= (uint32_t)(bi & 0xFF) << (8 * t);
    }
    // element 4l + t: sub-block j = l / 8, k-group g = (l % 8) / 2, byte
    // 4 (l % 2) + t of the group's 8
    const int j = l >> 3, g = (l & 7) >> 1;
    int8_t* fb = o.frag + sb * 4096 + 8 * j + 4 * (l & 1);
    *(uint32_t*)(fb + (16 * g + m) * 64) = pa;
    *(uint32_t*)(fb + (16 * g + 8 + m) * 64) = pb;
#pragma unroll
    for (int s = 1; s < 4; s <<= 1) {
        sa += __shfl_xor(sa, s, 64);
        sbb += __shfl_xor(sbb, s, 64);
    }
    if ((l & 3) == 0) {
        const int s16 = l >> 2;
        int8_t* x16 = o.xs16 + sb * 512;
        x16[m * 32 + s16] = (int8_t)(sa & 63);
        x16[m * 32 + 16 + s16] = (int8_t)(sa >> 6);
        x16[(8 + m) * 32 + s16] = (int8_t)(sbb & 63);
        x16[(8 + m) * 32 + 16 + s16] = (int8_t)(sbb >> 6);
    }
    sa += __shfl_xor(sa, 4, 64);
    sbb += __shfl_xor(sbb, 4, 64);
    if ((l & 7) == 0) {
        int8_t* x32 = o.xs32 + sb * 256;
        x32[m * 16 + j] = (int8_t)(sa & 63);
        x32[m * 16 + 8 + j] = (int8_t)(sa >> 6);
        x32[(8 + m) * 16 + j] = (int8_t)(sbb & 63);
        x32[(8 + m) * 16 + 8 + j] = (int8_t)(sbb >> 6);
    }
}
