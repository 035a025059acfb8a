/* libtinyinfer_host_codec.so — host INT8 weight codec.
 * Replaces reference backend/include/tinyinfer_host_codec.h:9-22 (definitions
 * at reference backend/host_codec.cpp:58-103).  Host-only, synchronous, no
 * allocation; all validation happens before any output byte is written.
 *  ti_host_quantize_f16: f16 bits [K,N] (N = columns = output channels) ->
 *    int8 q [K,N] in [-127,127] and fp32 scales [N]; scale[n] =
 *    float(double(max_k |w|) / 127) or 1.0 for an all-zero column;
 *    q = clamp(round_half_even(double(w) / double(scale[n])), -127, 127).
 *  ti_host_dequantize_i8: fp16_rn(float(q) * scale[n]); rejects -128,
 *    non-finite or non-positive scales and values that overflow binary16. */
#ifndef TINYINFER_HOST_CODEC_H
#define TINYINFER_HOST_CODEC_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
enum ti_host_status { TI_HOST_OK = 0, TI_HOST_INVALID = 1, TI_HOST_INTERNAL = 2 };
int ti_host_codec_abi_version(void); /* 1 */
int ti_host_quantize_f16(const uint16_t* f16_bits, size_t elements, size_t columns, int8_t* q,
                         size_t q_elements, float* scales, size_t scale_elements);
int ti_host_dequantize_i8(const int8_t* q, size_t elements, size_t columns, const float* scales,
                          size_t scale_elements, uint16_t* f16_bits, size_t output_elements);
#ifdef __cplusplus
}
#endif
#endif
