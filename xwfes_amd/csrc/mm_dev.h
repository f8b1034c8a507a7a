// mm_dev.h -- operand helpers shared by the fp16-MFMA kernels (k_gemm.hip,
// k_moe.hip): vector types, exact integer -> fp16 conversions and the fp16
// hi + lo split of an fp32 value.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

__device__ __forceinline__ v8h ld8h(const _Float16* p) { return *(const v8h*)p; }

// 8 nibbles (slot t: byte t % 4, nibble t / 4) -> fp16 q - bias, exact
__device__ __forceinline__ v8h nib8(uint32_t w, float bias) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    // 0x64 in the high byte: fp16 1024 + q
    const uint32_t p0 = __builtin_amdgcn_perm(lo, 0x64646464u, 0x00050004u);
    const uint32_t p1 = __builtin_amdgcn_perm(lo, 0x64646464u, 0x00070006u);
    const uint32_t p2 = __builtin_amdgcn_perm(hi, 0x64646464u, 0x00050004u);
    const uint32_t p3 = __builtin_amdgcn_perm(hi, 0x64646464u, 0x00070006u);
    const v2h b = {(_Float16)(-1024.f - bias), (_Float16)(-1024.f - bias)};
    const v2h h0 = __builtin_bit_cast(v2h, p0) + b, h1 = __builtin_bit_cast(v2h, p1) + b;
    const v2h h2 = __builtin_bit_cast(v2h, p2) + b, h3 = __builtin_bit_cast(v2h, p3) + b;
    return v8h{h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
}

// 8 signed bytes -> fp16 q, exact: (q ^ 0x80) = q + 128 as the low byte of
// fp16 1024 + q + 128, then - 1152
__device__ __forceinline__ v8h i8x8(v2i w) {
    const uint32_t a = (uint32_t)w.x ^ 0x80808080u, b = (uint32_t)w.y ^ 0x80808080u;
    const uint32_t p0 = __builtin_amdgcn_perm(a, 0x64646464u, 0x00050004u);
    const uint32_t p1 = __builtin_amdgcn_perm(a, 0x64646464u, 0x00070006u);
    const uint32_t p2 = __builtin_amdgcn_perm(b, 0x64646464u, 0x00050004u);
    const uint32_t p3 = __builtin_amdgcn_perm(b, 0x64646464u, 0x00070006u);
    const v2h o = {(_Float16)(-1152.f), (_Float16)(-1152.f)};
    const v2h h0 = __builtin_bit_cast(v2h, p0) + o, h1 = __builtin_bit_cast(v2h, p1) + o;
    const v2h h2 = __builtin_bit_cast(v2h, p2) + o, h3 = __builtin_bit_cast(v2h, p3) + o;
    return v8h{h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
}

// The hardware deals a launch's workgroups to the 8 XCDs in turn (linear
// workgroup id modulo 8), and each XCD has its own L2.  xcd_order maps the
// linear id to a logical index under which every XCD owns one contiguous run
// (XCD x: ids x, x + 8, x + 16, .. -> run x, in dispatch order), so that
// workgroups whose logical indices are neighbours (the token tiles of one
// weight tile) run on one XCD and share its L2.  A bijection of [0, total).
__device__ __forceinline__ uint32_t xcd_order(uint32_t lin, uint32_t total) {
    const uint32_t per = total >> 3, rem = total & 7, x = lin & 7, i = lin >> 3;
    return (x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per) + i;
}

// slot of element (token m, contraction k) in the one-pass GEMM's fragment-
// order operand planes ([Mp / 16][K / 32][64 lanes][8]; inter: each octet
// as its even then its odd elements, for Q4_0 weights)
__device__ __forceinline__ int64_t frag_at(int64_t m, int64_t k, int64_t K, bool inter) {
    const int64_t mt = m >> 4, ks = k >> 5;
    const int lane = (int)(m & 15) + 16 * (int)((k & 31) >> 3);
    int e = (int)(k & 7);
    if (inter) e = (e & 1) ? 4 + (e >> 1) : (e >> 1);
    return ((mt * (K / 32) + ks) * 64 + lane) * 8 + e;
}

// slot of the 32-element sum j of token m (the Q4_K min term's operand,
// [Mp / 16][K / 256][32 lanes][4])
__device__ __forceinline__ int64_t frag_sum_at(int64_t m, int64_t j, int64_t K) {
    const int64_t sb = j / 8;
    const int jj = (int)(j % 8);
    const int lane = (int)(m & 15) + 16 * (jj >> 2);
    return (((m >> 4) * (K / 256) + sb) * 32 + lane) * 4 + (jj & 3);
}

__device__ __forceinline__ void split_hl(float v, _Float16& h, _Float16& l) {
#pragma clang fp contract(off)
    h = (_Float16)v;
    l = (_Float16)(v - (float)h);
}

// split_hl of a pair, packed: both hi halves in one conversion, each lo half
// fp16(v - hi) by a mixed-precision fma that reads the hi half in place
// (v - hi is exact in fp32, so the result equals split_hl's)
__device__ __forceinline__ void split_hl2(float v0, float v1, v2h& h, v2h& l) {
    h = v2h{(_Float16)v0, (_Float16)v1};
    const uint32_t hw = __builtin_bit_cast(uint32_t, h);
    uint32_t lw;  // mixlo writes the low half, mixhi then the high half
    asm volatile("v_fma_mixlo_f16 %0, -%1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(lw) : "v"(hw), "v"(v0));
    asm volatile("v_fma_mixhi_f16 %0, -%1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
                 : "+v"(lw) : "v"(hw), "v"(v1));
    l = __builtin_bit_cast(v2h, lw);
}

}  // namespace
