/*
 * popcorn_safetensors.h — safetensors weight archives for the MI355X build.
 *
 * Replaces the archive the reference's example app opens through its
 * MTLSafeTensors dependency (Examples/GemmaCLI/Sources/GemmaCLI/
 * Gemma4TextInference.swift:22, `device.makeSafeTensors(from:)`) and reads in
 * Gemma4WeightLoader.swift:48-128 (`archive.names`, `archive.tensor(named:)`,
 * the dtype and shape of each tensor). The file is mapped read-only; its
 * header is parsed and validated once at open; tensors are copied from the
 * mapping to host or device memory by name. Device copies land in buffers
 * the caller allocated (popcorn_malloc aligns to 256 bytes), so the 4-byte
 * re-alignment the reference makes for packed u32 weights
 * (Gemma4WeightLoader.swift:67-78, :99-105) is never needed.
 *
 * Status codes as in popcorn_hip.h; a malformed archive or an unknown name is
 * -1100 with a message naming the problem.
 */
#ifndef POPCORN_SAFETENSORS_H
#define POPCORN_SAFETENSORS_H

#include "popcorn_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct popcorn_safetensors_s *popcorn_safetensors_t;

typedef struct {
    char name[256];
    char dtype_name[16];     /* the archive's name: "BF16", "U32", "F64", ...        */
    int32_t dtype;           /* POPCORN_DTYPE_*, or -1 (F64, F8_*: no tensor dtype)  */
    int32_t rank;
    int64_t shape[POPCORN_MAX_RANK];
    uint64_t offset;         /* byte offset in the data buffer                       */
    uint64_t nbytes;
    int32_t index;           /* position in the header                               */
} popcorn_safetensors_info_t;

/* Maps `path` and validates the header: length within the file and the
 * format's 100 MB limit, JSON object of entries {dtype, shape, data_offsets}
 * plus an optional "__metadata__" of strings, byte counts equal to
 * elements x dtype size, tensors tiling the data buffer. */
popcorn_status_t popcorn_safetensors_open(const char *path, popcorn_safetensors_t *archive);
popcorn_status_t popcorn_safetensors_close(popcorn_safetensors_t archive);

/* Number of tensors (SafeTensors.names.count), and each by header position. */
int32_t popcorn_safetensors_count(popcorn_safetensors_t archive);
popcorn_status_t popcorn_safetensors_info(popcorn_safetensors_t archive, int32_t index, popcorn_safetensors_info_t *info);
/* SafeTensors.tensor(named:)'s lookup; -1100 when absent. */
popcorn_status_t popcorn_safetensors_find(popcorn_safetensors_t archive, const char *name, popcorn_safetensors_info_t *info);
/* A "__metadata__" value (NUL-terminated into `value`). */
popcorn_status_t popcorn_safetensors_metadata(popcorn_safetensors_t archive, const char *key, char *value, size_t capacity);

/* Copies a tensor's bytes to host memory, or to device memory on `stream`
 * (returns once the mapping has been read). `capacity` is the destination's
 * size in bytes. Tensors of dtype -1 are refused (-1010). */
popcorn_status_t popcorn_safetensors_read(popcorn_safetensors_t archive, const char *name, void *dst, size_t capacity);
popcorn_status_t popcorn_safetensors_upload(popcorn_safetensors_t archive, const char *name, void *device_dst,
                                            size_t capacity, popcorn_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif
