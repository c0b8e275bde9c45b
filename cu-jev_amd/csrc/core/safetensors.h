/* Read-only view of every *.safetensors shard in a checkpoint directory.
 * Files are mmap'd; tensors point into the maps. Role of REF
 * src/core/safetensors.h:9-37 (format: 8-byte little-endian header length,
 * JSON header {name: {dtype, shape, data_offsets}}, then the data). */
#ifndef CUJEV_SAFETENSORS_H
#define CUJEV_SAFETENSORS_H

#include "cujev.h"
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum { ST_BF16 = 0, ST_F16 = 1, ST_F32 = 2, ST_OTHER = 3 } st_dtype;

typedef struct st_tensor {
    const char *name;
    st_dtype dtype;
    int ndim;
    int64_t shape[8];
    size_t numel;     /* product of shape */
    const void *data; /* inside the mmap */
    size_t nbytes;
} st_tensor;

typedef struct st_file st_file;

typedef struct st_bundle {
    st_file **files;
    int num_files;
    st_tensor *tensors; /* in file order */
    int num_tensors;
    int32_t *slots;     /* open-addressing index: tensor number or -1 */
    uint32_t slot_mask; /* slot count - 1 (a power of two, >= 2 x tensors) */
} st_bundle;

/* Maps every *.safetensors of `dir` and indexes their tensors by name; a name
 * that appears twice is a FORMAT error. */
cujev_status st_bundle_open(const char *dir, st_bundle *out);
void st_bundle_release(st_bundle *b);
/* The tensor called `name`, or NULL. */
const st_tensor *st_lookup(const st_bundle *b, const char *name);

#ifdef __cplusplus
}
#endif
#endif
