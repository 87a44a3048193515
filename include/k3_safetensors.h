#ifndef K3_SAFETENSORS_H
#define K3_SAFETENSORS_H

/*
 * Tensor-directory types of Moonshine's k3_safetensors.h (lines 1-58 there),
 * declared here with identical layout because k3_prefill_plan_build takes
 * the engine's k3_st_model as it is. Only the types: libk3moe reads the
 * directory (tensor names sorted by strcmp, as k3_st_model_open leaves
 * them) and never opens files. When the engine's own k3_safetensors.h is
 * included first, its identical definitions are used (same include guard).
 */

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#define K3_ST_MAX_DIMS 8

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    K3_ST_DTYPE_UNKNOWN = 0,
    K3_ST_DTYPE_BF16,
    K3_ST_DTYPE_F32,
    K3_ST_DTYPE_U8,
} k3_st_dtype;

typedef struct {
    char        *name;
    uint64_t     physical_offset;
    uint64_t     byte_length;
    uint64_t     shape[K3_ST_MAX_DIMS];
    uint16_t     shard;
    uint8_t      ndim;
    k3_st_dtype  dtype;
} k3_st_tensor;

typedef struct {
    char     *path;
    int       fd;
    int       direct_fd;
    uint64_t  file_bytes;
    uint64_t  data_offset;
} k3_st_shard;

typedef struct {
    k3_st_shard  *shards;
    size_t        shard_count;
    k3_st_tensor *tensors;
    size_t        tensor_count;
    size_t        tensor_capacity;
} k3_st_model;

#ifdef __cplusplus
}
#endif

#endif
