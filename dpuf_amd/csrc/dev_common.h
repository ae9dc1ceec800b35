// dev_common.h -- gfx950 device helpers of the DPUF engine's HIP code: fp16
// scales, the reference's hsum trees and exp polynomial, FWHT-64 in registers
// and over lane quads, the activation prep (int8 quantisation per 32-block)
// and the exact u4 x i8 row-block dot.
#ifndef DPUF_DEV_COMMON_H
#define DPUF_DEV_COMMON_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hip_layer.h"

#define DEV __device__ __forceinline__

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Scalar helpers
// ---------------------------------------------------------------------------
DEV float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// 8-lane sum in the order of the reference's eng_hsum256_ps
// (dpuf_engine.c:37-46): ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)).
DEV float hsum8(const float* a) {
    float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
    return (s0 + s1) + (s2 + s3);
}

// 8-lane sum as hsum4_256_ps's hadd tree leaves it (dpuf_engine.c:318-323):
// ((a0+a1)+(a2+a3)) + ((a4+a5)+(a6+a7)).
DEV float hsum8_hadd(const float* a) {
    float lo = (a[0] + a[1]) + (a[2] + a[3]);
    float hi = (a[4] + a[5]) + (a[6] + a[7]);
    return lo + hi;
}

// The reference's own 8-wide exp polynomial (dpuf_engine.c:297-316), per lane.
DEV float exp_poly(float x) {
    x = fmaxf(-45.0f, fminf(x, 45.0f));
    float fx = rintf(x * 1.44269504088896341f);
    float r = fmaf(-fx, 0.693359375f, x);
    r = fmaf(-fx, -2.12194440e-4f, r);
    float p = 1.9875691500e-4f;
    p = fmaf(p, r, 1.3981999507e-3f);
    p = fmaf(p, r, 8.3334519073e-3f);
    p = fmaf(p, r, 4.1665795894e-2f);
    p = fmaf(p, r, 1.6666665459e-1f);
    p = fmaf(p, r, 5.0000001201e-1f);
    float r2 = r * r;
    float er = fmaf(p, r2, r) + 1.0f;
    int n = (int)fx;
    return er * __int_as_float((n + 127) << 23);
}


// In-register FWHT-64: radix-2 butterflies with strides 1..32, then x 1/8
// (reference fwht64_block_f32, dpuf_avx2.c:724-772).
DEV void fwht64(float* y) {
#pragma unroll
    for (int h = 1; h < 64; h <<= 1) {
#pragma unroll
        for (int i = 0; i < 64; i += 2 * h) {
#pragma unroll
            for (int j = i; j < i + h; j++) {
                float a = y[j], b = y[j + h];
                y[j] = a + b;
                y[j + h] = a - b;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 64; i++) y[i] = y[i] * 0.125f;
}

// DPP quad permutations: xor 1 = (1,0,3,2), xor 2 = (2,3,0,1).
DEV int dpp_xor1(int v) { return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false); }
DEV int dpp_xor2(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false); }


// ---------------------------------------------------------------------------
// Activation prep spread over lane quads.
//
// A 64-column block is owned by 4 consecutive lanes (a quad); quarter qp
// holds columns 16*qp .. 16*qp+15 in registers.  FWHT stages with strides
// 1, 2, 4, 8 run inside the lane, stride 16 pairs lanes qp and qp^1, stride
// 32 pairs qp and qp^2 (DPP quad permutes).  Every butterfly is the same
// single a+b / a-b as in the reference (dpuf_avx2.c:724-772) and the stages
// keep its ascending order, so results are bit-identical.  Lanes (0,1) and
// (2,3) of a quad then quantise one 32-block each
// (dpuf_prep_had4_packed_slab, dpuf_avx2.c:2400-2446).
// ---------------------------------------------------------------------------
struct PrepSet {
    const uint8_t* sign[3];
    DpufPrep p[3];
    int n;
};

DEV float fxor1(float v) { return __int_as_float(dpp_xor1(__float_as_int(v))); }
DEV float fxor2(float v) { return __int_as_float(dpp_xor2(__float_as_int(v))); }

// Maximum over the 64 lanes, in every lane: DPP inside each 16-lane row
// (xor 1, xor 2, half-row mirror, row mirror), then the four rows' values
// read into scalars.  fmaxf is exact, so the grouping is free.
DEV float wave_max(float v) {
    v = fmaxf(v, fxor1(v));
    v = fmaxf(v, fxor2(v));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// ---------------------------------------------------------------------------
// Activation prep of one 64-block by one wave, lane l holding column l: the
// latency-bound form for a few blocks at the end of a kernel.
//
// FWHT stride h pairs lane l with l ^ h: DPP quad permutes for h = 1, 2,
// row rotations for 4 and 8 (row_ror:N hands lane i the value of lane
// (i - N) mod 16, so l ^ 4 is ror 4 for lanes with bit 2 set and ror 12
// for the others, and l ^ 8 is ror 8), shuffles for 16 and 32.  Each
// butterfly is the reference's a + b / a - b with a the lower column, in
// ascending stride order, so the values equal quad_fwht64's.  The 32-block
// maximum and the integer sum (both order-free) use the same moves.
// ---------------------------------------------------------------------------
#define DPP_F(v, ctrl) __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xF, 0xF, false))
#define DPP_I(v, ctrl) __builtin_amdgcn_update_dpp(0, (v), ctrl, 0xF, 0xF, false)

DEV void wave_prep64(float x, int lane, int blk, int8_t* q, float* s, int32_t* m, uint16_t* h) {
    // FWHT-64 across the wave
    {
        float p = DPP_F(x, 0xB1);  // l ^ 1
        x = (lane & 1) ? p - x : x + p;
        p = DPP_F(x, 0x4E);  // l ^ 2
        x = (lane & 2) ? p - x : x + p;
        const float r4 = DPP_F(x, 0x124), r12 = DPP_F(x, 0x12C);
        p = (lane & 4) ? r4 : r12;  // l ^ 4
        x = (lane & 4) ? p - x : x + p;
        p = DPP_F(x, 0x128);  // l ^ 8
        x = (lane & 8) ? p - x : x + p;
        p = __shfl_xor(x, 16, 64);
        x = (lane & 16) ? p - x : x + p;
        p = __shfl_xor(x, 32, 64);
        x = (lane & 32) ? p - x : x + p;
        x = x * 0.125f;
    }
    // maximum of |x| over the lane's 32-block
    float amax = fabsf(x);
    amax = fmaxf(amax, DPP_F(amax, 0xB1));
    amax = fmaxf(amax, DPP_F(amax, 0x4E));
    amax = fmaxf(amax, DPP_F(amax, 0x124));
    amax = fmaxf(amax, DPP_F(amax, 0x128));
    amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
    int32_t qi = 0;
    float d = 0.0f;
    if (!(amax <= 1e-4f)) {
        d = amax / 127.0f;
        const float inv = (amax > 1e-12f) ? (127.0f / amax) : 0.0f;
        const float xs = x * inv;
        if (!(xs > -2147483648.0f && xs < 2147483648.0f)) qi = -127;  // cvtps -> INT_MIN -> -127
        else qi = (int32_t)rintf(xs);
        qi = qi > 127 ? 127 : qi;
        qi = qi < -127 ? -127 : qi;
    }
    int32_t sum = qi;
    sum += DPP_I(sum, 0xB1);
    sum += DPP_I(sum, 0x4E);
    sum += DPP_I(sum, 0x124);
    sum += DPP_I(sum, 0x128);
    sum += __shfl_xor(sum, 16, 64);
    q[64 * blk + lane] = (int8_t)qi;
    if (h) h[64 * blk + lane] = __builtin_bit_cast(uint16_t, (_Float16)qi);
    if ((lane & 31) == 0) {
        s[2 * blk + (lane >> 5)] = d;
        m[2 * blk + (lane >> 5)] = sum * 8;
    }
}

// Sign bits of the lane's 16 columns of 64-block blk (bit c%8 of byte c/8
// set = negate column c).
DEV uint32_t quad_sign_bits(const uint8_t* sign, int blk, int qp) {
    return sign ? *(const uint16_t*)(sign + 8 * blk + 2 * qp) : 0u;
}

DEV void apply_sign_bits(float* v, uint32_t sb) {
#pragma unroll
    for (int k = 0; k < 16; k++)
        if ((sb >> k) & 1u) v[k] = -v[k];
}

DEV void quad_fwht64(float* v, int qp) {
#pragma unroll
    for (int h = 1; h < 16; h <<= 1) {
#pragma unroll
        for (int i = 0; i < 16; i += 2 * h) {
#pragma unroll
            for (int j = i; j < i + h; j++) {
                const float a = v[j], b = v[j + h];
                v[j] = a + b;
                v[j + h] = a - b;
            }
        }
    }
    const bool lo1 = (qp & 1) == 0, lo2 = (qp & 2) == 0;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const float p = fxor1(v[j]);
        v[j] = lo1 ? v[j] + p : p - v[j];
    }
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const float p = fxor2(v[j]);
        v[j] = lo2 ? v[j] + p : p - v[j];
    }
#pragma unroll
    for (int j = 0; j < 16; j++) v[j] = v[j] * 0.125f;
}

// Quantises the lane's 16 FWHT'd values (half of 32-block 2*blk + qp/2) and
// stores the int8 values, and from the even lane the block scale and 8*sum(q).
typedef _Float16 gm_h2 __attribute__((ext_vector_type(2)));

// Two fp16 values from bytes b0, b1 of x and 0x64: 1024 + byte each.
DEV uint32_t gm_pair(uint32_t x, uint32_t sel) { return __builtin_amdgcn_perm(0x64646464u, x, sel); }

DEV uint32_t gm_sub(uint32_t v, _Float16 c) {
    gm_h2 h = __builtin_bit_cast(gm_h2, v);
    h = h - (gm_h2){c, c};
    return __builtin_bit_cast(uint32_t, h);
}

// Four int8 (one word) -> four f16 in two words (exact).
DEV void i8x4_to_h(uint32_t x, uint32_t& a, uint32_t& b) {
    const uint32_t u = x ^ 0x80808080u;  // q + 128 per byte
    a = gm_sub(gm_pair(u, 0x04010400u), (_Float16)1152.0f);
    b = gm_sub(gm_pair(u, 0x04030402u), (_Float16)1152.0f);
}

// Activation prep of one 64-block by the 16 lanes of a DPP row, lane r of
// the row holding columns 4r .. 4r + 3 in x[0..3]: FWHT strides 1 and 2
// inside the lane, strides 4, 8, 16, 32 between lanes r ^ 1, r ^ 2, r ^ 4,
// r ^ 8 (the moves of wave_prep64), the same butterflies in the same order
// as quad_fwht64; then the quantisation of quad_quant_store with the
// 32-block (lanes 0-7 or 8-15 of the row) maximum and sum over r ^ 1, r ^ 2
// and the half-row mirror.  All 16 lanes of the row must be active.  COH:
// q, s and m are written with agent-scope stores (they go past the L2 to
// where every XCD reads, for readers in the same launch).
template <bool COH = false>
DEV void row_prep64(float* x, int r, int blk, int8_t* q, float* s, int32_t* m, uint16_t* h) {
    {
        float a = x[0], b = x[1];
        x[0] = a + b;
        x[1] = a - b;
        a = x[2];
        b = x[3];
        x[2] = a + b;
        x[3] = a - b;
        a = x[0];
        b = x[2];
        x[0] = a + b;
        x[2] = a - b;
        a = x[1];
        b = x[3];
        x[1] = a + b;
        x[3] = a - b;
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float p = DPP_F(x[k], 0xB1);  // column stride 4: lane r ^ 1
        x[k] = (r & 1) ? p - x[k] : x[k] + p;
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float p = DPP_F(x[k], 0x4E);  // stride 8: r ^ 2
        x[k] = (r & 2) ? p - x[k] : x[k] + p;
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float r4 = DPP_F(x[k], 0x124), r12 = DPP_F(x[k], 0x12C);  // stride 16: r ^ 4
        const float p = (r & 4) ? r4 : r12;
        x[k] = (r & 4) ? p - x[k] : x[k] + p;
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float p = DPP_F(x[k], 0x128);  // stride 32: r ^ 8
        x[k] = (r & 8) ? p - x[k] : x[k] + p;
    }
#pragma unroll
    for (int k = 0; k < 4; k++) x[k] = x[k] * 0.125f;
    float amax = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
    amax = fmaxf(amax, DPP_F(amax, 0xB1));
    amax = fmaxf(amax, DPP_F(amax, 0x4E));
    amax = fmaxf(amax, DPP_F(amax, 0x141));
    int32_t qi[4] = {0, 0, 0, 0};
    float d = 0.0f;
    if (!(amax <= 1e-4f)) {
        d = amax / 127.0f;
        const float inv = (amax > 1e-12f) ? (127.0f / amax) : 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float xs = x[k] * inv;
            int32_t v;
            if (!(xs > -2147483648.0f && xs < 2147483648.0f)) v = -127;  // cvtps -> INT_MIN -> -127
            else v = (int32_t)rintf(xs);
            v = v > 127 ? 127 : v;
            qi[k] = v < -127 ? -127 : v;
        }
    }
    int32_t sum = (qi[0] + qi[1]) + (qi[2] + qi[3]);
    sum += DPP_I(sum, 0xB1);
    sum += DPP_I(sum, 0x4E);
    sum += DPP_I(sum, 0x141);
    const uint32_t w = (uint32_t)(qi[0] & 0xFF) | ((uint32_t)(qi[1] & 0xFF) << 8) | ((uint32_t)(qi[2] & 0xFF) << 16) |
                       ((uint32_t)(qi[3] & 0xFF) << 24);
    if (COH) {
        __hip_atomic_store((uint32_t*)(q + 64 * blk + 4 * r), w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((r & 7) == 0) {
            __hip_atomic_store((uint32_t*)(s + 2 * blk + (r >> 3)), __float_as_uint(d), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(m + 2 * blk + (r >> 3), sum * 8, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }
    *(uint32_t*)(q + 64 * blk + 4 * r) = w;
    if (h) {
        uint32_t a, b;
        i8x4_to_h(w, a, b);
        *(uint2*)(h + 64 * blk + 4 * r) = make_uint2(a, b);
    }
    if ((r & 7) == 0) {
        s[2 * blk + (r >> 3)] = d;
        m[2 * blk + (r >> 3)] = sum * 8;
    }
}


DEV void quad_quant_store(const float* v, int qp, int blk, int8_t* q, float* s, int32_t* m, uint16_t* h) {
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const float a = fabsf(v[k]);
        amax = a > amax ? a : amax;
    }
    const float other = fxor1(amax);
    amax = other > amax ? other : amax;
    uint32_t w[4] = {0u, 0u, 0u, 0u};
    int32_t sum = 0;
    float d = 0.0f;
    if (!(amax <= 1e-4f)) {
        d = amax / 127.0f;
        const float inv = (amax > 1e-12f) ? (127.0f / amax) : 0.0f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float x = v[4 * g + k] * inv;
                int32_t qi;
                if (!(x > -2147483648.0f && x < 2147483648.0f)) qi = -127;  // cvtps -> INT_MIN -> -127
                else qi = (int32_t)rintf(x);
                qi = qi > 127 ? 127 : qi;
                qi = qi < -127 ? -127 : qi;
                sum += qi;
                w[g] |= ((uint32_t)(qi & 0xFF)) << (8 * k);
            }
        }
    }
    sum += dpp_xor1(sum);
    *(uint4*)(q + 64 * blk + 16 * qp) = make_uint4(w[0], w[1], w[2], w[3]);
    if (h) {  // the same 16 values as fp16 (exact: |q| <= 127)
        uint32_t hw[8];
#pragma unroll
        for (int g = 0; g < 4; g++) i8x4_to_h(w[g], hw[2 * g], hw[2 * g + 1]);
        *(uint4*)(h + 64 * blk + 16 * qp) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        *(uint4*)(h + 64 * blk + 16 * qp + 8) = make_uint4(hw[4], hw[5], hw[6], hw[7]);
    }
    if ((qp & 1) == 0) {
        s[2 * blk + (qp >> 1)] = d;
        m[2 * blk + (qp >> 1)] = sum * 8;
    }
}

DEV void load16(const float* p, float* v) {
    const float4* p4 = (const float4*)p;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 t = p4[i];
        v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
}

DEV void store16(float* p, const float* v) {
    float4* p4 = (float4*)p;
#pragma unroll
    for (int i = 0; i < 4; i++) p4[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
}


// Exact integer dot of one row block: 32 nibbles u in [0, 15] against 32 int8
// activations (x as 8 words, word 2c = columns 8c..8c+3, word 2c+1 = 8c+4..8c+7).
// Equals the reference's maddubs/madd sum (dpuf_avx2.c:2623-2632), whose int16
// partials cannot overflow (|sum| <= 30480).
DEV int row_block_dot(uint4 w, int4 xa, int4 xb) {
    const uint32_t m = 0x0F0F0F0Fu;
    int d = __builtin_amdgcn_sdot4((int)(w.x & m), xa.x, 0, false);
    d = __builtin_amdgcn_sdot4((int)((w.x >> 4) & m), xa.y, d, false);
    d = __builtin_amdgcn_sdot4((int)(w.y & m), xa.z, d, false);
    d = __builtin_amdgcn_sdot4((int)((w.y >> 4) & m), xa.w, d, false);
    d = __builtin_amdgcn_sdot4((int)(w.z & m), xb.x, d, false);
    d = __builtin_amdgcn_sdot4((int)((w.z >> 4) & m), xb.y, d, false);
    d = __builtin_amdgcn_sdot4((int)(w.w & m), xb.z, d, false);
    d = __builtin_amdgcn_sdot4((int)((w.w >> 4) & m), xb.w, d, false);
    return d;
}



// The same for a mode 14 row block: bits 4..5 of each value come from the
// row's two words of high bits (word c >> 1, bits (c & 1) * 4 + {0,1} of byte
// k for column 8c+k, + {2,3} for 8c+4+k).  u <= 63, so the sdot4 products are
// exact, as the reference's maddubs sums (dpuf_avx2.c:2824-2846).
DEV int row_block_dot6(uint4 w, uint2 hw, int4 xa, int4 xb) {
    const uint32_t m = 0x0F0F0F0Fu, m2 = 0x03030303u;
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
    const int xw[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    int d = 0;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t h = ((c >> 1) ? hw.y : hw.x) >> ((c & 1) * 4);
        const uint32_t lo = (wd[c] & m) | ((h & m2) << 4);
        const uint32_t hi = ((wd[c] >> 4) & m) | (((h >> 2) & m2) << 4);
        d = __builtin_amdgcn_sdot4((int)lo, xw[2 * c], d, false);
        d = __builtin_amdgcn_sdot4((int)hi, xw[2 * c + 1], d, false);
    }
    return d;
}

// Lane i + 8 of a 16-lane row for lane i and the reverse (DPP row_ror:8).
DEV int dpp_ror8(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false); }

DEV uint4 nt_load16(const uint8_t* p) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Top-2 with multiplicity (the reference's sequential b1/b2 scan,
// dpuf_engine.c:2101-2110, is order independent), then the early-exit
// decision b1 - b2 >= thr (thr > 0).
// (Selects, not branches: with branches the compiler merged the two
// conditional stores into a store through a selected address, which kept
// the pair in scratch.)
DEV void top2_take(float v, float& b1, float& b2) {
    const bool g1 = v > b1, g2 = v > b2;
    const float n2 = g1 ? b1 : (g2 ? v : b2);
    b1 = g1 ? v : b1;
    b2 = n2;
}

DEV void top2_merge(float& b1, float& b2, float c1, float c2) {
    if (b1 >= c1) {
        b2 = fmaxf(b2, c1);
    } else {
        b2 = fmaxf(c2, b1);
        b1 = c1;
    }
}

// First maximum (dpuf-cli.c:1997-2004: `if (x[i] > best)` from best = x[0]):
// the larger value, the smaller index on ties; every partial starts from
// (x[0], 0), so a NaN x[0] gives 0 as the reference does and other NaNs are
// never taken.
DEV void amax_merge(float& bv, int& bi, float v, int i) {
    const bool take = v > bv || (v == bv && i < bi);
    bv = take ? v : bv;
    bi = take ? i : bi;
}

// A partial of the LM-head reductions over some rows of a logit row:
// (top-1, top-2, first-max value, its row as int bits).  Top-2 starts from
// -1e30 as the scan over the whole row does; the first maximum from (-inf,
// INT_MAX), so that merging partials in any order gives the smallest row of
// the largest value and never a NaN (a NaN logit 0 is the caller's case).
// A native vector: the HIP float4 struct would be kept in scratch.
typedef float lm4 __attribute__((ext_vector_type(4)));
DEV lm4 lm_part_init() { return (lm4){-1e30f, -1e30f, __int_as_float(0xFF800000), __int_as_float(0x7FFFFFFF)}; }
DEV lm4 lm_part_take(lm4 p, float v, int row) {
    float b1 = p[0], b2 = p[1], av = p[2];
    int bi = __float_as_int(p[3]);
    top2_take(v, b1, b2);
    amax_merge(av, bi, v, row);
    return (lm4){b1, b2, av, __int_as_float(bi)};
}
DEV lm4 lm_part_merge(lm4 p, lm4 o) {
    float b1 = p[0], b2 = p[1], av = p[2];
    int bi = __float_as_int(p[3]);
    top2_merge(b1, b2, o[0], o[1]);
    amax_merge(av, bi, o[2], __float_as_int(o[3]));
    return (lm4){b1, b2, av, __int_as_float(bi)};
}
// The merge of a wave's 64 partials, in every lane.
DEV lm4 lm_part_wave(lm4 p) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const lm4 q = {__shfl_xor(p[0], o, 64), __shfl_xor(p[1], o, 64), __shfl_xor(p[2], o, 64),
                       __shfl_xor(p[3], o, 64)};
        p = lm_part_merge(p, q);
    }
    return p;
}

// 4 x 4 transpose of (16-lane row, register): afterwards register j of lane
// row g holds what register g of lane row j held.
DEV void skp_transpose(uint32_t& r0, uint32_t& r1, uint32_t& r2, uint32_t& r3) {
    // rows 2, 3 of r0 <-> rows 0, 1 of r2; the same for r1, r3
    const auto a = __builtin_amdgcn_permlane32_swap(r0, r2, false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(r1, r3, false, false);
    // rows 1, 3 of the first <-> rows 0, 2 of the second
    const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
    const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    r0 = c[0];
    r1 = c[1];
    r2 = d[0];
    r3 = d[1];
}



// LDS address space pointer of the direct-to-LDS loads.
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Vector types of the MFMA kernels.
typedef _Float16 gm_h8 __attribute__((ext_vector_type(8)));
typedef float gm_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t gm_u4 __attribute__((ext_vector_type(4)));

// Lane t of one row: columns 4t .. 4t + 3 of the 64-block t / 16 (COH: see
// row_prep64).
// One element of the SwiGLU with dead zone (reference swiglu_range_avx2,
// 8-wide path, dpuf_engine.c:976-989), then the down input's sign bit.
DEV float swiglu1(float g, float u, float dz, uint32_t neg) {
    const float ng = fmaxf(-40.0f, fminf(0.0f - g, 40.0f));
    const float silu = g / (1.0f + exp_poly(ng));
    float rr = silu * u;
    if (dz > 0.0f && !(fabsf(rr) >= dz)) rr = 0.0f;
    return neg ? -rr : rr;
}

template <bool COH = false>
DEV void swiglu_prep_lane(int I, const float* __restrict__ gate, const float* __restrict__ up, float dz,
                          const uint8_t* __restrict__ sign, int8_t* q, float* s, int32_t* m, uint16_t* h, int t) {
    const int blk = t >> 4, r = t & 15;
    const float4 g4 = *(const float4*)(gate + 4 * t);
    const float4 u4 = *(const float4*)(up + 4 * t);
    const uint32_t sb = sign ? (sign[8 * blk + (r >> 1)] >> (4 * (r & 1))) & 0xFu : 0u;
    const float g[4] = {g4.x, g4.y, g4.z, g4.w}, u[4] = {u4.x, u4.y, u4.z, u4.w};
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; k++) v[k] = swiglu1(g[k], u[k], dz, (sb >> k) & 1u);
    row_prep64<COH>(v, r, blk, q, s, m, h);
}

// The plain prep of lane t of one row (columns 4t .. 4t + 3): sign, then
// row_prep64 (COH: see row_prep64).
template <bool COH = false>
DEV void prep_lane(const float* __restrict__ x, const uint8_t* __restrict__ sign, int8_t* q, float* s, int32_t* m, int t) {
    const int blk = t >> 4, r = t & 15;
    const float4 x4 = *(const float4*)(x + 4 * t);
    const uint32_t sb = sign ? (sign[8 * blk + (r >> 1)] >> (4 * (r & 1))) & 0xFu : 0u;
    float v[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
    for (int k = 0; k < 4; k++) v[k] = ((sb >> k) & 1u) ? -v[k] : v[k];
    row_prep64<COH>(v, r, blk, q, s, m, nullptr);
}

// Records the first HIP error of the current API call (rt.hip).
void dpuf_note(hipError_t e, const char* what);

#endif
