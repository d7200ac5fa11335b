/*
 * gguf.h -- GGUF v2/v3 container: tensor descriptors and model metadata.
 *
 * Drop-in for the reference interface include/gguf.h:1-120.  The type ids,
 * the descriptor fields and the metadata record are the GGUF/ggml on-disk
 * contract, so names and layouts match the reference; the implementation
 * (host/gguf.c) is this library's own.
 */
#if !defined(QWEN_GGUF_H) && !defined(GGUF_H)   /* either header, whichever came first */
#define QWEN_GGUF_H
/* the reference header of the same name is superseded by this one when both
   are on the include path (reference drivers compiled against this library) */
#define GGUF_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GGUF_MAGIC 0x46554747u            /* "GGUF" little-endian */
#define GGUF_DEFAULT_ALIGNMENT 32
#define GGUF_MAX_NAME 64

/* metadata value types (GGUF spec) -- reference gguf.h:10-24 */
typedef enum {
    GGUF_TYPE_UINT8 = 0, GGUF_TYPE_INT8 = 1, GGUF_TYPE_UINT16 = 2, GGUF_TYPE_INT16 = 3,
    GGUF_TYPE_UINT32 = 4, GGUF_TYPE_INT32 = 5, GGUF_TYPE_FLOAT32 = 6, GGUF_TYPE_BOOL = 7,
    GGUF_TYPE_STRING = 8, GGUF_TYPE_ARRAY = 9, GGUF_TYPE_UINT64 = 10, GGUF_TYPE_INT64 = 11,
    GGUF_TYPE_FLOAT64 = 12,
} gguf_type_t;

typedef struct {
    uint32_t magic;
    uint32_t version;
    uint64_t tensor_count;
    uint64_t metadata_kv_count;
} __attribute__((packed)) gguf_header_t;

/* ggml tensor element formats (ggml numbering) -- reference gguf.h:37-61 */
typedef enum {
    GGML_F32 = 0, GGML_F16 = 1, GGML_Q4_0 = 2, GGML_Q4_1 = 3, GGML_Q5_0 = 6, GGML_Q5_1 = 7,
    GGML_Q8_0 = 8, GGML_Q2_K = 10, GGML_Q3_K = 11, GGML_Q4_K = 12, GGML_Q5_K = 13,
    GGML_Q6_K = 14, GGML_Q8_K = 15, GGML_IQ2_XXS = 16, GGML_IQ2_XS = 17, GGML_IQ3_XXS = 18,
    GGML_IQ1_S = 19, GGML_IQ4_NL = 20, GGML_IQ3_S = 21, GGML_IQ2_S = 22, GGML_IQ4_XS = 23,
    GGML_IQ1_M = 24, GGML_BF16 = 25,
} ggml_type_t;

/* one tensor: ne[0] is the contiguous (input) dimension, ne[1] the rows */
typedef struct {
    char         name[GGUF_MAX_NAME];
    uint32_t     n_dims;
    uint64_t     ne[4];
    ggml_type_t  type;
    uint64_t     offset;      /* relative to the data section */
    const void  *data;        /* host address of the tensor bytes */
} gguf_tensor_info_t;

/* model hyper-parameters read from "<arch>.*" keys -- reference gguf.h:72-94 */
typedef struct {
    uint32_t n_embd, n_head, n_head_kv, head_dim, n_layer, n_ff, vocab_size, context_len;
    float    rope_theta;
    uint32_t rope_dim_count;
    uint32_t rope_sections[4];
    float    rms_norm_eps;
    bool     tie_word_embeddings;
    uint32_t full_attn_interval, ssm_state_size, ssm_conv_kernel, ssm_inner_size,
             ssm_group_count, nextn_layers;
} qwen_config_t;

typedef struct {
    int                 fd;
    size_t              file_size;
    const void         *mmap_data;
    const void         *data_base;
    uint32_t            alignment;
    char                arch[32];
    gguf_header_t       header;
    qwen_config_t       config;
    gguf_tensor_info_t *tensors;
    uint64_t            tensor_count;
} gguf_context_t;

/* Opens and parses a GGUF file (mmap).  0 on success, -1 on failure
 * (message on stderr).  Replaces reference gguf.c:185-310. */
int  gguf_open(gguf_context_t *ctx, const char *filepath);
/* Unmaps and frees.  Replaces reference gguf.c:174-183. */
void gguf_close(gguf_context_t *ctx);
/* Byte size of a fixed-size metadata type, 0 for string/array (gguf.c:14-29). */
size_t gguf_type_size(gguf_type_t t);
/* Exact-name lookup, NULL if absent (gguf.c:312-317). */
const gguf_tensor_info_t *gguf_find_tensor(const gguf_context_t *ctx, const char *name);

#ifdef __cplusplus
}
#endif
#endif
