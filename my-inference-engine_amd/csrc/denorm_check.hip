/*
 * Build-time guard (see the Makefile): compiled with exactly the flags of
 * qmv_kernels.hip, this kernel's descriptor must keep fp32 and fp16/fp64
 * denormals (float_denorm_mode 3). The single-position Q4_K/Q6_K paths feed
 * 4-bit codes to v_fma_mix_f32 as fp16 subnormals (q * 2^-24) and keep sums
 * scaled by 2^-24, so a build that flushes denormals
 * (-fgpu-flush-denormals-to-zero, -ffast-math) would silently zero them.
 */
#include <hip/hip_runtime.h>

__global__ void denorm_mode_probe(float *out, const _Float16 *in)
{
    out[threadIdx.x] = (float)in[threadIdx.x] * 0.5f;
}
