/*
 * zl_gguf -- GGUF model files to device tables (C-ABI, part of libhip_bridge.so).
 *
 * ziglm reads GGUF in Zig (src/gguf.zig GGUFFile) and uploads each weight to its own
 * device buffer (src/cuda_model.zig:24-57, 237-337). This header replaces that pair for a
 * host written in any language: a reader with the same accept/reject behaviour, getters
 * and parameter extraction as GGUFFile, and a staged uploader that moves tensor bytes
 * into caller-owned device buffers. Each entry point cites the Zig declaration it
 * replaces as "gguf.zig:LINE" (or types.zig / cuda_model.zig).
 *
 * File layout (GGUF v2 / v3, all integers little endian):
 *   u32 magic 0x46554747 ("GGUF"), u32 version, u64 tensor_count, u64 metadata_count,
 *   metadata_count x { string key, u32 value_type, value },
 *   tensor_count  x { string name, u32 n_dims (<= 4), u64 dims[n_dims], u32 ggml_type,
 *                     u64 offset },
 *   padding to general.alignment (default 32), then tensor data; tensor i starts at
 *   data_offset + offset_i.  string = u64 length + bytes (no terminator); array value =
 *   u32 element type + u64 count + elements.
 *
 * Borrowing: every pointer handed out (names, keys, string values, tensor data) points
 * into the mapped file (or the caller's buffer for zl_gguf_open_buffer) and stays valid
 * until zl_gguf_close. Names and keys are not NUL-terminated: use the *_len fields.
 * The reader never touches the GPU; only the upload entry points do.
 */
#ifndef ZL_GGUF_H
#define ZL_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "hip_bridge.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Open / parse errors: one code per error the Zig reader returns. */
#define ZL_GGUF_OK 0
#define ZL_GGUF_EOPEN (-10)            /* file cannot be opened / mapped / read (errno kept) */
#define ZL_GGUF_EINVALID_FILE (-11)    /* InvalidGGUFFile: shorter than 24 bytes (gguf.zig:80) */
#define ZL_GGUF_EMAGIC (-12)           /* InvalidGGUFMagic (gguf.zig:246) */
#define ZL_GGUF_EVERSION (-13)         /* UnsupportedGGUFVersion: not 2 or 3 (gguf.zig:250-252) */
#define ZL_GGUF_EEOF (-14)             /* UnexpectedEOF: a field runs past the end (gguf.zig:159-205) */
#define ZL_GGUF_EVALUE_TYPE (-15)      /* UnsupportedGGUFValueType: type id > 12 (gguf.zig:236) */
#define ZL_GGUF_EDIMS (-16)            /* InvalidTensorDimensions: n_dims > 4 (gguf.zig:276) */
#define ZL_GGUF_EOUT_OF_BOUNDS (-17)   /* TensorDataOutOfBounds (gguf.zig:307-309) */
#define ZL_GGUF_EALIGNMENT (-18)       /* new: general.alignment 0 or not a power of two */
#define ZL_GGUF_ENOMEM (-19)           /* allocation failed */
#define ZL_GGUF_EINVAL (-20)           /* bad argument (NULL handle, index out of range, ...) */
#define ZL_GGUF_ESIZE (-21)            /* upload: destination smaller than the tensor */

/* GGUFValueType (gguf.zig:11-26). */
#define ZL_GGUF_UINT8 0
#define ZL_GGUF_INT8 1
#define ZL_GGUF_UINT16 2
#define ZL_GGUF_INT16 3
#define ZL_GGUF_UINT32 4
#define ZL_GGUF_INT32 5
#define ZL_GGUF_FLOAT32 6
#define ZL_GGUF_BOOL 7
#define ZL_GGUF_STRING 8
#define ZL_GGUF_ARRAY 9
#define ZL_GGUF_UINT64 10
#define ZL_GGUF_INT64 11
#define ZL_GGUF_FLOAT64 12

/* Architecture (types.zig:211-223, same order). */
#define ZL_ARCH_LLAMA 0
#define ZL_ARCH_QWEN2 1
#define ZL_ARCH_MISTRAL 2
#define ZL_ARCH_GEMMA 3
#define ZL_ARCH_GEMMA2 4
#define ZL_ARCH_GEMMA4 5
#define ZL_ARCH_PHI 6
#define ZL_ARCH_PHI3 7
#define ZL_ARCH_DEEPSEEK 8
#define ZL_ARCH_STARCODER2 9
#define ZL_ARCH_GPT2 10
#define ZL_ARCH_UNKNOWN 11

typedef struct ZlGguf ZlGguf;

/* One metadata entry (GGUFMetadataKV, gguf.zig:50-53). `data` points at the value bytes
 * as stored: scalars little endian; STRING: the bytes after the length (data_bytes = the
 * length); ARRAY: the elements after the u32 type and u64 count. */
typedef struct {
    const char* key;
    uint64_t key_len;
    uint32_t type;       /* ZL_GGUF_* */
    uint32_t array_type; /* element type when type == ZL_GGUF_ARRAY, else 0 */
    uint64_t array_len;  /* element count when type == ZL_GGUF_ARRAY, else 0 */
    const void* data;
    uint64_t data_bytes;
} ZlGgufKV;

/* One tensor (types.zig:296-302 Tensor). shape[] holds dims in GGUF order (shape[0] is
 * the contiguous one), 1 past n_dims. size_bytes = (elements / block_size) * type_size
 * with the block and type sizes of types.zig:33-67 (zl_ggml_block_size/type_size). */
typedef struct {
    const char* name;
    uint64_t name_len;
    uint32_t type; /* GGMLType id (types.zig:4-31; HIP_BRIDGE_Q4_0 etc. are the same ids) */
    uint32_t n_dims;
    uint64_t shape[4];
    uint64_t offset; /* relative to the data section */
    const void* data;
    uint64_t size_bytes;
} ZlGgufTensor;

/* ModelParams (types.zig:246-267) as extracted by GGUFFile.extractParams
 * (gguf.zig:399-451) and completed by initComputed (types.zig:269-285). */
typedef struct {
    int32_t arch; /* ZL_ARCH_* */
    int32_t use_gemma_rms_unit_offset;
    uint64_t context_length;
    uint64_t embedding_length;
    uint64_t feed_forward_length;
    uint64_t head_count;
    uint64_t head_count_kv;
    uint64_t block_count;
    uint64_t head_size;
    uint64_t vocab_size;
    float layer_norm_rms_epsilon;
    float rope_freq_base;
    float rope_freq_scale;
    float attn_logit_softcapping;
    float final_logit_softcapping;
    int32_t rope_type; /* 0 normal (half split), 1 neox */
    uint64_t rope_dim_count;
    uint64_t expert_count;
    uint64_t expert_used_count;
    uint64_t sliding_window;
    uint64_t num_kv_shared_layers;
} ZlModelParams;

/* ---- open / close ------------------------------------------------------------------- */
/* Map `path` read-only and parse it (GGUFFile.open, gguf.zig:73-110; a failed mmap falls
 * back to reading the file into memory, as the reference). *out is NULL on error. */
int zl_gguf_open(const char* path, ZlGguf** out);                          /* gguf.zig:73 */
/* Parse a caller-owned buffer that must outlive the handle (GGUFFile.initFromBuffer). */
int zl_gguf_open_buffer(const void* data, uint64_t size, ZlGguf** out);    /* gguf.zig:113 */
void zl_gguf_close(ZlGguf* f);                                             /* gguf.zig:138 */
/* Name of a ZL_GGUF_* code ("InvalidGGUFMagic", ...), as the Zig error names. */
const char* zl_gguf_error_name(int code);

/* ---- header ------------------------------------------------------------------------- */
uint32_t zl_gguf_version(const ZlGguf* f);        /* GGUFFile.version */
uint64_t zl_gguf_tensor_count(const ZlGguf* f);   /* GGUFFile.tensor_count */
uint64_t zl_gguf_metadata_count(const ZlGguf* f); /* GGUFFile.metadata_count */
uint64_t zl_gguf_alignment(const ZlGguf* f);      /* GGUFFile.alignment */
uint64_t zl_gguf_data_offset(const ZlGguf* f);    /* GGUFFile.data_offset */
uint64_t zl_gguf_file_size(const ZlGguf* f);      /* raw_buffer.len */
const void* zl_gguf_base(const ZlGguf* f);        /* raw_buffer.ptr */

/* ---- metadata ----------------------------------------------------------------------- */
int zl_gguf_metadata(const ZlGguf* f, uint64_t index, ZlGgufKV* out);
/* Index of the first entry whose key equals `key` (getMetadata's linear scan,
 * gguf.zig:319-324), or -1. */
int64_t zl_gguf_find_metadata(const ZlGguf* f, const char* key);
/* Typed getters (gguf.zig:326-389): return 1 and store the value when the key exists
 * with a convertible type, else 0. Conversions as the reference: u32 from UINT32, UINT64
 * (truncated), INT32; u64 from UINT64, UINT32, INT64, INT32 and from the first element of
 * an array of those; f32 from FLOAT32, FLOAT64 and the first element of a FLOAT32 array.
 * A negative INT32 / INT64 (which the reference rejects with a panic) gives 0. */
int zl_gguf_get_u32(const ZlGguf* f, const char* key, uint32_t* out);      /* gguf.zig:326 */
int zl_gguf_get_u64(const ZlGguf* f, const char* key, uint64_t* out);      /* gguf.zig:338 */
int zl_gguf_get_f32(const ZlGguf* f, const char* key, float* out);         /* gguf.zig:364 */
int zl_gguf_get_string(const ZlGguf* f, const char* key, const char** s, uint64_t* len); /* gguf.zig:382 */

/* ---- tensors ------------------------------------------------------------------------ */
int zl_gguf_tensor(const ZlGguf* f, uint64_t index, ZlGgufTensor* out);
/* Index of the tensor named `name` (the last one of that name, as the reference's
 * tensor_map), or -1; fills *out when found and out != NULL. */
int64_t zl_gguf_find_tensor(const ZlGguf* f, const char* name, ZlGgufTensor* out); /* gguf.zig:391 */
/* Block and byte sizes of a GGML type (types.zig:33-67, including its fallbacks for
 * types it does not size: block 32 or 256, type size 1). */
uint64_t zl_ggml_block_size(uint32_t type);                                /* types.zig:33 */
uint64_t zl_ggml_type_size(uint32_t type);                                 /* types.zig:42 */

/* ---- parameters --------------------------------------------------------------------- */
void zl_gguf_params(const ZlGguf* f, ZlModelParams* out);                  /* gguf.zig:399 */

/* ---- device tables -------------------------------------------------------------------- */
/* Copy the bytes of tensors indices[0..n) into dsts[0..n) (device buffers of at least
 * dst_bytes[i] bytes, hip_malloc'd by the caller, as CudaGpuTensor.upload's buffers,
 * cuda_model.zig:24-36). The bytes go through a ring of pinned host slots: host threads
 * copy from the mapped file into a slot while the DMA engine drains the previous ones,
 * ordered on `stream`. Returns when every copy has completed (0), or the first error
 * (ZL_GGUF_EINVAL / ZL_GGUF_ESIZE before any copy; a hipError_t value). */
int zl_gguf_upload_tensors(const ZlGguf* f, const uint64_t* indices, void* const* dsts,
                           const uint64_t* dst_bytes, uint64_t n, HipStream_t stream);
/* One tensor (cuda_model.zig:24 CudaGpuTensor.upload / 47 CudaGpuNorm.upload). */
int zl_gguf_upload(const ZlGguf* f, uint64_t index, void* dst, uint64_t dst_bytes,
                   HipStream_t stream);
/* Copy `bytes` from any host memory to the device through the same pinned ring. */
int zl_upload_host(void* dst, const void* src, uint64_t bytes, HipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* ZL_GGUF_H */
