"""Test helper: the per-matrix entry points of include/k3_rocm_ops.h
(k3_rocm_ops.h of the reference) called on torch device tensors.

Each function keeps the reference's name, argument order and meaning and
returns the C launcher's bool (False = invalid arguments, nothing launched).
`stream` defaults to torch's current stream. Everything runs in
libk3moe.so (gfx950 HIP); there is no other path.
"""
import ctypes

from moonshine_amd._lib import lib


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is not None:
        return ctypes.c_void_p(stream)
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def k3_rocm_situ_bf16(output, gate, up, element_count, beta, linear_beta, stream=None):
    return lib().k3_rocm_situ_bf16(_ptr(output), _ptr(gate), _ptr(up), element_count, beta,
                                   linear_beta, _stream(stream))


def k3_rocm_swiglu_bf16(output, gate, up, element_count, stream=None):
    return lib().k3_rocm_swiglu_bf16(_ptr(output), _ptr(gate), _ptr(up), element_count,
                                     _stream(stream))


def k3_rocm_mxfp4_gemv_bf16(output, packed, scales, input, rows, columns, stream=None):
    return lib().k3_rocm_mxfp4_gemv_bf16(_ptr(output), _ptr(packed), _ptr(scales), _ptr(input),
                                         rows, columns, _stream(stream))


def k3_rocm_mxfp4_gemm_bf16(output, packed, scales, input, vector_count, rows, columns,
                            stream=None):
    return lib().k3_rocm_mxfp4_gemm_bf16(_ptr(output), _ptr(packed), _ptr(scales), _ptr(input),
                                         vector_count, rows, columns, _stream(stream))


def k3_rocm_mxfp4_gemm_tiled_bf16(output, packed, scales, input, vector_count, rows, columns,
                                  batch_tile, stream=None):
    return lib().k3_rocm_mxfp4_gemm_tiled_bf16(_ptr(output), _ptr(packed), _ptr(scales),
                                               _ptr(input), vector_count, rows, columns,
                                               batch_tile, _stream(stream))


def k3_rocm_bf16_gemv_f32(output, weights, input, rows, columns, stream=None):
    return lib().k3_rocm_bf16_gemv_f32(_ptr(output), _ptr(weights), _ptr(input), rows, columns,
                                       _stream(stream))


def k3_rocm_bf16_gemm_f32(output, weights, input, vector_count, rows, columns, stream=None):
    return lib().k3_rocm_bf16_gemm_f32(_ptr(output), _ptr(weights), _ptr(input), vector_count,
                                       rows, columns, _stream(stream))


def k3_rocm_bf16_gemm_tiled_f32(output, weights, input, vector_count, rows, columns,
                                batch_tile, stream=None):
    return lib().k3_rocm_bf16_gemm_tiled_f32(_ptr(output), _ptr(weights), _ptr(input),
                                             vector_count, rows, columns, batch_tile,
                                             _stream(stream))


def k3_rocm_rms_norm_bf16(output, input, weight, vector_count, hidden_size, epsilon,
                          stream=None):
    return lib().k3_rocm_rms_norm_bf16(_ptr(output), _ptr(input), _ptr(weight), vector_count,
                                       hidden_size, epsilon, _stream(stream))


def k3_rocm_bf16_gemv_bf16(output, weights, input, rows, columns, stream=None):
    return lib().k3_rocm_bf16_gemv_bf16(_ptr(output), _ptr(weights), _ptr(input), rows, columns,
                                        _stream(stream))


def k3_rocm_bf16_gemm_bf16(output, weights, input, vector_count, rows, columns, stream=None):
    return lib().k3_rocm_bf16_gemm_bf16(_ptr(output), _ptr(weights), _ptr(input), vector_count,
                                        rows, columns, _stream(stream))


def k3_rocm_bf16_gemm_tiled_bf16(output, weights, input, vector_count, rows, columns,
                                 batch_tile, stream=None):
    return lib().k3_rocm_bf16_gemm_tiled_bf16(_ptr(output), _ptr(weights), _ptr(input),
                                              vector_count, rows, columns, batch_tile,
                                              _stream(stream))


def k3_rocm_bf16_quantize_q8_128(quantized, scales, weights, rows, columns, stream=None):
    return lib().k3_rocm_bf16_quantize_q8_128(_ptr(quantized), _ptr(scales), _ptr(weights), rows,
                                              columns, _stream(stream))


def k3_rocm_q8_128_dequantize_bf16(weights, quantized, scales, rows, columns, stream=None):
    return lib().k3_rocm_q8_128_dequantize_bf16(_ptr(weights), _ptr(quantized), _ptr(scales),
                                                rows, columns, _stream(stream))


def k3_rocm_q8_128_gemv_bf16(output, quantized, scales, input, rows, columns, stream=None):
    return lib().k3_rocm_q8_128_gemv_bf16(_ptr(output), _ptr(quantized), _ptr(scales),
                                          _ptr(input), rows, columns, _stream(stream))


def k3_rocm_q8_128_gemm_bf16(output, quantized, scales, input, vector_count, rows, columns,
                             stream=None):
    return lib().k3_rocm_q8_128_gemm_bf16(_ptr(output), _ptr(quantized), _ptr(scales),
                                          _ptr(input), vector_count, rows, columns,
                                          _stream(stream))


def k3_rocm_q8_128_gemm_tiled_bf16(output, quantized, scales, input, vector_count, rows,
                                   columns, batch_tile, stream=None):
    return lib().k3_rocm_q8_128_gemm_tiled_bf16(_ptr(output), _ptr(quantized), _ptr(scales),
                                                _ptr(input), vector_count, rows, columns,
                                                batch_tile, _stream(stream))


def k3_rocm_router_topk_f32(expert_ids, expert_weights, logits, correction_bias, expert_count,
                            top_k, scaling_factor, stream=None):
    return lib().k3_rocm_router_topk_f32(_ptr(expert_ids), _ptr(expert_weights), _ptr(logits),
                                         _ptr(correction_bias), expert_count, top_k,
                                         scaling_factor, _stream(stream))


def k3_rocm_router_topk_f32_batch(expert_ids, expert_weights, logits, correction_bias,
                                  vector_count, expert_count, top_k, scaling_factor,
                                  stream=None):
    return lib().k3_rocm_router_topk_f32_batch(_ptr(expert_ids), _ptr(expert_weights),
                                               _ptr(logits), _ptr(correction_bias),
                                               vector_count, expert_count, top_k,
                                               scaling_factor, _stream(stream))


def k3_rocm_weighted_sum_bf16(output, vectors, weights, vector_count, hidden_size, stream=None):
    return lib().k3_rocm_weighted_sum_bf16(_ptr(output), _ptr(vectors), _ptr(weights),
                                           vector_count, hidden_size, _stream(stream))


def k3_rocm_weighted_sum_bf16_batch(output, vectors, weights, token_count, vector_count,
                                    hidden_size, stream=None):
    return lib().k3_rocm_weighted_sum_bf16_batch(_ptr(output), _ptr(vectors), _ptr(weights),
                                                 token_count, vector_count, hidden_size,
                                                 _stream(stream))


def k3_rocm_gather_rows_bf16(output, input, row_ids, row_count, row_size, stream=None):
    return lib().k3_rocm_gather_rows_bf16(_ptr(output), _ptr(input), _ptr(row_ids), row_count,
                                          row_size, _stream(stream))


def k3_rocm_scatter_rows_bf16(output, input, row_ids, row_count, row_size, stream=None):
    return lib().k3_rocm_scatter_rows_bf16(_ptr(output), _ptr(input), _ptr(row_ids), row_count,
                                           row_size, _stream(stream))


def k3_rocm_add_bf16(output, left, right, element_count, stream=None):
    return lib().k3_rocm_add_bf16(_ptr(output), _ptr(left), _ptr(right), element_count,
                                  _stream(stream))
