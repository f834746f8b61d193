// The reference's kernel-level API (include/forge/matmul_neon.hpp:20-92)
// with host pointers, computed on the GPU through libpocketforge_amd.so (a
// per-thread device context, created on first use).
#ifndef FORGE_MATMUL_NEON_HPP
#define FORGE_MATMUL_NEON_HPP

#include <cstdint>
#include <vector>

#include "types.hpp"

namespace forge {

void quantize_activation_row(const float* src, int8_t* dst, float* scale_out, uint32_t n);

// Load-time unpack of packed codes (the device kernels unpack in registers).
void dequant_q4_to_int8(const uint8_t* q4_data, int8_t* i8_data, float scale, uint32_t n);
void dequant_q2_to_int8(const uint8_t* q2_data, int8_t* i8_data, float scale, uint32_t n);
void dequant_ternary_to_int8(const uint8_t* t_data, int8_t* i8_data, uint32_t n);

// C = A * B^T, A int8 [M x K], B int8 [N x K], C int32 [M x N].
void matmul_int8(const int8_t* A, const int8_t* B, int32_t* C, uint32_t M, uint32_t N, uint32_t K);

// C = (float)(quantize(A) * B^T) * act_scale[i] * weight_scale[j].
void matmul_quantized(const float* A, const int8_t* B, float* C, uint32_t M, uint32_t N, uint32_t K,
                      const float* weight_scales, const float* act_scales);

float dot_product(const float* a, const float* b, uint32_t n);
void softmax(float* vals, uint32_t n);
void rmsnorm(float* out, const float* x, const float* weight, uint32_t n);

}  // namespace forge
#endif
