// Device-side helpers shared by the gfx950 kernels: bf16 conversion, 16-byte
// vector moves and the MFMA operand types.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "awa_plan.h"

namespace s2 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// The reference round_bf16 (adaptive_window_attention.cpp:499-508), returning
// the upper 16 bits: round to nearest even; for Inf/NaN the increment is
// skipped, so a NaN whose payload sits only in the low 16 bits becomes Inf,
// exactly as on the reference CPU path.
__device__ __forceinline__ uint16_t round_bf16_ref_bits(float x) {
    uint32_t b = __float_as_uint(x);
    if ((b & 0x7f800000u) != 0x7f800000u) b += 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}

// Storage conversion fp32 -> bf16: round to nearest even, NaN stays NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
    uint32_t b = __float_as_uint(x);
    if ((b & 0x7f800000u) == 0x7f800000u)
        return (uint16_t)((b >> 16) | ((b & 0xffffu) ? 0x40u : 0u));
    b += 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}

// two floats -> packed bf16 pair (low, high) with the hardware conversion
// (v_cvt_pk_bf16_f32, round to nearest even; equal to f32_to_bf16 for every
// non-NaN input)
__device__ __forceinline__ uint32_t pack2_bf16_rne(float lo, float hi) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)lo) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)hi) << 16);
}

// Storage conversion fp32 -> fp16, round to nearest even, of x as rounded to
// fp32.  The empty asm keeps the compiler from folding the conversion into
// the fma, add or multiply that produced x (a v_fma_mix*_f16 rounds the exact
// result once, which differs from rounding to fp32 and then to fp16 when the
// fp32 value lies on an fp16 midpoint).
__device__ __forceinline__ _Float16 f32_to_f16(float x) {
    asm("" : "+v"(x));
    return (_Float16)x;
}

// two floats -> packed fp16 pair (low, high), round to nearest even
__device__ __forceinline__ uint32_t pack2_f16_rne(float lo, float hi) {
    return (uint32_t)__builtin_bit_cast(uint16_t, f32_to_f16(lo)) |
           ((uint32_t)__builtin_bit_cast(uint16_t, f32_to_f16(hi)) << 16);
}

// Four consecutive floats stored at element `idx` of an activation buffer of
// element type `kind` (0 fp32, 1 bf16, 2 fp16; the s2_dtype values).
__device__ __forceinline__ void store4(void* base, long idx, float a, float b, float c, float d,
                                       int kind) {
    if (kind == 1) {
        *reinterpret_cast<uint2*>((uint16_t*)base + idx) =
            make_uint2(pack2_bf16_rne(a, b), pack2_bf16_rne(c, d));
    } else if (kind == 2) {
        *reinterpret_cast<uint2*>((uint16_t*)base + idx) =
            make_uint2(pack2_f16_rne(a, b), pack2_f16_rne(c, d));
    } else {
        *reinterpret_cast<float4*>((float*)base + idx) = make_float4(a, b, c, d);
    }
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(((uint32_t)h) << 16);
}

// Load 8 consecutive elements as fp32.
__device__ __forceinline__ void load8(const uint16_t* p, float (&v)[8]) {
    const uint4 raw = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}

__device__ __forceinline__ void load8(const float* p, float (&v)[8]) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

__device__ __forceinline__ uint4 pack8_bf16(const uint16_t (&h)[8]) {
    uint4 r;
    r.x = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
    r.y = (uint32_t)h[2] | ((uint32_t)h[3] << 16);
    r.z = (uint32_t)h[4] | ((uint32_t)h[5] << 16);
    r.w = (uint32_t)h[6] | ((uint32_t)h[7] << 16);
    return r;
}

// eight floats to bf16 (round to nearest even), as four pair conversions
// (v_cvt_pk_bf16_f32), packed in element order
__device__ __forceinline__ uint4 cvt8_bf16(const float (&x)[8]) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const f32x2_t f = {x[2 * i], x[2 * i + 1]};
        w[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) {
    return __builtin_bit_cast(bf16x8, v);
}

// Raw buffer descriptor over [base, base + bytes): loads past the end return
// zero.  Word 3 is the gfx950 descriptor format for untyped dword access.
typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ i32x4 buffer_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = (uint64_t)base;
    i32x4 r;
    r.x = (int)(uint32_t)a;
    r.y = (int)(uint32_t)(a >> 32);   // stride 0: raw buffer
    r.z = (int)bytes;                 // num_records
    r.w = 0x00020000;
    return r;
}

// A descriptor the compiler cannot prove wave-uniform (built from values
// that passed through control flow) moved to SGPRs; the caller guarantees
// that every lane holds the same value.
__device__ __forceinline__ i32x4 wave_uniform(i32x4 r) {
    r.x = __builtin_amdgcn_readfirstlane(r.x);
    r.y = __builtin_amdgcn_readfirstlane(r.y);
    r.z = __builtin_amdgcn_readfirstlane(r.z);
    r.w = __builtin_amdgcn_readfirstlane(r.w);
    return r;
}

// One buffer_load_dwordx4 with the lds modifier: lane i's 16 bytes land at
// LDS address lds_addr + 16*i (lds_addr wave-uniform).  Issued through asm
// so that the compiler does not order every later LDS read behind it: the
// caller waits for the data with s_waitcnt vmcnt and a barrier.  M0 is
// written only by this helper in these kernels.
__device__ __forceinline__ void lds_dma16(i32x4 rsrc, uint32_t lds_addr, uint32_t voffset,
                                          uint32_t soffset) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(lds_addr), "v"(voffset), "s"(rsrc), "s"(soffset)
                 : "memory", "m0");
}

// Physical workgroup id -> logical id such that consecutive logical ids run
// on the same XCD (the hardware deals workgroups to XCDs round-robin).
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
    const int xcd = bid % kNumXcd;
    const int idx = bid / kNumXcd;
    const int per = nblocks / kNumXcd;
    const int rem = nblocks % kNumXcd;
    return xcd * per + (xcd < rem ? xcd : rem) + idx;
}

}  // namespace s2
