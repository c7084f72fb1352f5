// hw_probe.hip - writes what gfx950 instructions return, as golden vectors for the CPU oracle's restatements.
//
// Run once on an MI355X by make_hw_fixture.py (which builds this file with hipcc into tests/golden/_build/); the
// outputs are committed as tests/golden/hw_probe.npz and read by the CPU tests:
//   cvt    v_cvt_scalef32_pk_fp8_bf16 of every bf16 bit pattern at scale 1.0 and 0.25 (the P conversion)
//   pknorm v_cvt_pknorm_u16_f32 of a fixed set of f32 inputs (the Schraudolph exp2)
//   mfma   v_mfma_scale_f32_32x32x64_f8f6f4 (e4m3 x e4m3) on fixed operands, per-lane E8M0 scale bytes and C
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef short v2s __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

__global__ void probe_cvt(uint8_t* out) {   // out[2][65536]
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;   // 32768 threads, two bf16 patterns each
    const uint32_t lo = 2u * i, hi = 2u * i + 1u;
    const v2bf x = __builtin_bit_cast(v2bf, (uint32_t)(lo | (hi << 16)));
    const v2s a = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16((v2s){0, 0}, x, 1.0f, false);
    const v2s b = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16((v2s){0, 0}, x, 0.25f, false);
    const uint32_t wa = __builtin_bit_cast(uint32_t, a), wb = __builtin_bit_cast(uint32_t, b);
    out[lo] = (uint8_t)wa;
    out[hi] = (uint8_t)(wa >> 8);
    out[65536u + lo] = (uint8_t)wb;
    out[65536u + hi] = (uint8_t)(wb >> 8);
}

__global__ void probe_pknorm(const float* x, uint16_t* out, uint32_t n) {   // n even
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (2u * i + 1u >= n) return;
    const uint32_t w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pknorm_u16(x[2u * i], x[2u * i + 1u]));
    out[2u * i] = (uint16_t)w;
    out[2u * i + 1u] = (uint16_t)(w >> 16);
}

// One wave: a [64 lanes][8 dwords] A, b [64][8] B, sa / sb [64] scale dwords (op_sel 0: byte 0), c [64][16]
// -> d [64][16]. Operands are passed in the register layout; the test maps lanes to rows / columns.
__global__ void probe_mfma(const int* a, const int* b, const int* sa, const int* sb, const float* c, float* d) {
    const uint32_t l = threadIdx.x;
    v8i va, vb;
    v16f vc;
    for (int i = 0; i < 8; ++i) { va[i] = a[l * 8 + i]; vb[i] = b[l * 8 + i]; }
    for (int i = 0; i < 16; ++i) vc[i] = c[l * 16 + i];
    const v16f r = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(va, vb, vc, 0, 0, 0, sa[l], 0, sb[l]);
    for (int i = 0; i < 16; ++i) d[l * 16 + i] = r[i];
}

extern "C" int hw_probe_run(uint8_t* h_cvt, const float* h_px, uint16_t* h_pk, uint32_t n_pk, const int* h_a, const int* h_b,
                            const int* h_sa, const int* h_sb, const float* h_c, float* h_d) {
    uint8_t* d_cvt;
    float *d_px, *d_c, *d_d;
    uint16_t* d_pk;
    int *d_a, *d_b, *d_sa, *d_sb;
    if (hipMalloc(&d_cvt, 131072) || hipMalloc(&d_px, n_pk * 4) || hipMalloc(&d_pk, n_pk * 2) || hipMalloc(&d_a, 2048) ||
        hipMalloc(&d_b, 2048) || hipMalloc(&d_sa, 256) || hipMalloc(&d_sb, 256) || hipMalloc(&d_c, 4096) || hipMalloc(&d_d, 4096))
        return 1;
    (void)hipMemcpy(d_px, h_px, n_pk * 4, hipMemcpyHostToDevice);
    (void)hipMemcpy(d_a, h_a, 2048, hipMemcpyHostToDevice);
    (void)hipMemcpy(d_b, h_b, 2048, hipMemcpyHostToDevice);
    (void)hipMemcpy(d_sa, h_sa, 256, hipMemcpyHostToDevice);
    (void)hipMemcpy(d_sb, h_sb, 256, hipMemcpyHostToDevice);
    (void)hipMemcpy(d_c, h_c, 4096, hipMemcpyHostToDevice);
    hipLaunchKernelGGL(probe_cvt, dim3(128), dim3(256), 0, 0, d_cvt);
    hipLaunchKernelGGL(probe_pknorm, dim3((n_pk / 2 + 255) / 256), dim3(256), 0, 0, d_px, d_pk, n_pk);
    hipLaunchKernelGGL(probe_mfma, dim3(1), dim3(64), 0, 0, d_a, d_b, d_sa, d_sb, d_c, d_d);
    if (hipDeviceSynchronize()) return 2;
    (void)hipMemcpy(h_cvt, d_cvt, 131072, hipMemcpyDeviceToHost);
    (void)hipMemcpy(h_pk, d_pk, n_pk * 2, hipMemcpyDeviceToHost);
    (void)hipMemcpy(h_d, d_d, 4096, hipMemcpyDeviceToHost);
    (void)hipFree(d_cvt); (void)hipFree(d_px); (void)hipFree(d_pk); (void)hipFree(d_a); (void)hipFree(d_b); (void)hipFree(d_sa); (void)hipFree(d_sb); (void)hipFree(d_c); (void)hipFree(d_d);
    return hipGetLastError() == hipSuccess ? 0 : 3;
}
