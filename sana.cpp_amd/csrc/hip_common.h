// Shared device helpers for the gfx950 (MI355X) kernels of the Sana DiT path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define SANA_DEV __device__ __forceinline__

// 64-lane wavefront reductions (CDNA: wavefront = 64).
SANA_DEV float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

SANA_DEV float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

SANA_DEV float silu_f(float x) { return x / (1.0f + expf(-x)); }

// SiLU from the hardware v_exp_f32 (2^x) and v_rcp_f32, each good to ~1 ulp:
// x * 1 / (1 + 2^(-x log2 e)), 5 VALU ops instead of ~21 for expf and an IEEE
// divide.  For kernels whose result is rounded to fp16.  Limits match silu_f:
// x -> -inf gives -0 (2^+inf = inf, 1/inf = 0), x -> +inf gives x.
SANA_DEV float silu_fast(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

SANA_DEV float gelu_tanh_f(float x) {
    const float a = 0.7978845608028654f;  // sqrt(2/pi)
    return 0.5f * x * (1.0f + tanhf(a * (x + 0.044715f * x * x * x)));
}

// v_mfma_f32_32x32x16_f16 (gfx950): A lane l holds row l%32, k = 8*(l/32)+e;
// B lane l holds column l%32, k = 8*(l/32)+e; D lane l holds column l%32,
// rows 8*(r/4) + 4*(l/32) + r%4 for r = 0..15.
SANA_DEV f32x16 mfma_32x32x16(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_16x16x32_f16 (gfx950): A lane l holds row l%16, k = 8*(l/16)+e;
// B lane l holds column l%16, k = 8*(l/16)+e; D lane l holds column l%16,
// rows 4*(l/16) + r for r = 0..3.
SANA_DEV f32x4 mfma_16x16x32(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
