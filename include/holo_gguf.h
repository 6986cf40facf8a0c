/*
 * holo_gguf.h -- GGUF model files: parse, query, and upload every tensor to
 * MI355X HBM in one arena.
 *
 * The parser follows the reference's src/ai/gguf.c (privuser2738/google-classic)
 * exactly where the result depends on it, so a file reads the same way in
 * both:
 *   - magic "GGUF", versions 2 and 3 only (gguf.c:283-296);
 *   - strings of at most 1 MiB, arrays of at most 10,000,000 elements,
 *     at most 4 dimensions per tensor (gguf.c:147, 202, 336);
 *   - tensor names keep their first 255 bytes, up to a NUL (gguf.c:332);
 *   - size_bytes = (n_elements / block size) * block bytes, from the
 *     reference's type tables; types without an entry have size 0
 *     (gguf.c:26-71, 106-109, 351);
 *   - the tensor data section starts at the end of the tensor table rounded
 *     up to 32 bytes; general.alignment is not consulted (gguf.c:355-356);
 *   - the model parameters use the same keys and defaults (gguf.c:358-393);
 *     rope_freq_scale is never read and stays 0.
 *
 * Upload: holo_gguf_upload copies the whole tensor data section into one
 * device allocation through two pinned staging buffers on the library's copy
 * stream, so that file reads overlap the host-to-device copies.  Tensor
 * offsets inside the section are kept, so every tensor's device address is
 * the arena base plus its offset (32-byte aligned, as in the file).
 *
 * Parsing and the metadata calls touch no GPU state.
 */
#ifndef HOLO_GGUF_H
#define HOLO_GGUF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Value types of metadata (gguf.h:23-37); the numbering is the file format's. */
enum {
    HOLO_GGUF_UINT8 = 0, HOLO_GGUF_INT8 = 1, HOLO_GGUF_UINT16 = 2, HOLO_GGUF_INT16 = 3,
    HOLO_GGUF_UINT32 = 4, HOLO_GGUF_INT32 = 5, HOLO_GGUF_FLOAT32 = 6, HOLO_GGUF_BOOL = 7,
    HOLO_GGUF_STRING = 8, HOLO_GGUF_ARRAY = 9, HOLO_GGUF_UINT64 = 10, HOLO_GGUF_INT64 = 11,
    HOLO_GGUF_FLOAT64 = 12
};

typedef struct holo_gguf holo_gguf_t; /* opaque parsed file */

/* A string value as stored by the reference (gguf.h:77-80): the elements of a
 * string array returned by holo_gguf_get_array have this layout.           */
typedef struct {
    uint64_t len;
    char *data;
} holo_gguf_string_t;

/* One tensor of the file: the fields of gguf_tensor_info_t (gguf.h:107-118). */
typedef struct {
    char name[256];
    uint32_t n_dims;
    uint64_t dims[4];
    int32_t type;        /* GGML type number: 2 = Q4_0, 8 = Q8_0, 12 = Q4_K, ... */
    uint64_t offset;     /* from the start of the tensor data section */
    uint64_t n_elements;
    uint64_t size_bytes;
} holo_gguf_tensor_t;

/* Model parameters read from metadata (gguf.h:151-165). */
typedef struct {
    char arch[64];
    uint32_t vocab_size;
    uint32_t context_length;
    uint32_t embedding_length;
    uint32_t block_count;
    uint32_t attention_head_count;
    uint32_t attention_head_count_kv;
    uint32_t attention_key_length;
    uint32_t feed_forward_length;
    float rope_freq_base;
    float rope_freq_scale;
    float rms_norm_eps;
} holo_gguf_model_t;

/* gguf_open (gguf.c:266): NULL on any format error, with a message on stderr. */
holo_gguf_t *holo_gguf_open(const char *path);
/* gguf_close (gguf.c:402); also frees the device arena, if any.              */
void holo_gguf_close(holo_gguf_t *g);

uint32_t holo_gguf_version(const holo_gguf_t *g);
uint64_t holo_gguf_n_tensors(const holo_gguf_t *g);
uint64_t holo_gguf_n_kv(const holo_gguf_t *g);
uint64_t holo_gguf_data_offset(const holo_gguf_t *g);
const holo_gguf_model_t *holo_gguf_model(const holo_gguf_t *g);

/* Key i (0 <= i < n_kv), or NULL.                                            */
const char *holo_gguf_key(const holo_gguf_t *g, uint64_t i);
/* Value type of key, or -1 when absent (gguf_get_value, gguf.c:432).        */
int holo_gguf_value_type(const holo_gguf_t *g, const char *key);
/* gguf_get_string (gguf.c:443): NULL unless the value is a string.          */
const char *holo_gguf_get_string(const holo_gguf_t *g, const char *key);
/* gguf_get_int (gguf.c:451): integer types of up to 64 bits, else default.  */
int64_t holo_gguf_get_int(const holo_gguf_t *g, const char *key, int64_t default_val);
/* gguf_get_float (gguf.c:468): float32 or float64 (narrowed), else default. */
float holo_gguf_get_float(const holo_gguf_t *g, const char *key, float default_val);
/* gguf_get_array (gguf.c:479): element data and count; *elem_type (if not
 * NULL) receives the element type.  String arrays hold holo_gguf_string_t.  */
const void *holo_gguf_get_array(const holo_gguf_t *g, const char *key, uint64_t *len, int *elem_type);

/* Tensor i (0 <= i < n_tensors), or NULL.                                    */
const holo_gguf_tensor_t *holo_gguf_tensor(const holo_gguf_t *g, uint64_t i);
/* gguf_find_tensor (gguf.c:493).                                              */
const holo_gguf_tensor_t *holo_gguf_find_tensor(const holo_gguf_t *g, const char *name);
/* gguf_load_tensor (gguf.c:512): the tensor's size_bytes into a host buffer
 * of at least that size; 0 or -1.                                            */
int holo_gguf_load_tensor(holo_gguf_t *g, const holo_gguf_tensor_t *t, void *buffer, size_t size);

/* Copies the tensor data section (through the end of the last tensor) into
 * one device allocation; 0 or -1.  Replaces the per-tensor cuda_malloc +
 * cuda_memcpy_h2d of the reference's upload_tensor (llm_cuda.c:346-440).
 * Blocking: returns when the data is on the device.  A second call returns
 * the existing arena.                                                        */
int holo_gguf_upload(holo_gguf_t *g);
/* Device base of the arena and its size (NULL / 0 before the upload).        */
void *holo_gguf_device_base(const holo_gguf_t *g);
size_t holo_gguf_device_bytes(const holo_gguf_t *g);
/* Device address of a tensor: arena base + offset (NULL before the upload).  */
void *holo_gguf_device_ptr(const holo_gguf_t *g, const holo_gguf_tensor_t *t);

#ifdef __cplusplus
}
#endif

#endif /* HOLO_GGUF_H */
