/* A reader for GGUF version 3 model files (one file, or shards named "<stem>-0000i-of-0000N.gguf"), and a loader of
 * one MoE block's tensors from it into a context.
 *
 * Replaces the reference's core/load/gguf.h:12-78 (GgufTensor, GgufValue, GgufModel: metadata, a tensor table whose
 * bytes are mapped read-only, release of a tensor's pages, gguf_architecture, ggml_type_bytes), as C calls in the
 * conventions of c0ven_moe.h: a moe_status from every call, gguf_last_error for the message, plain structs. The file
 * format is GGUF v3 as ggml writes it (magic "GGUF", version 3, tensor and key counts, typed key/value pairs, tensor
 * infos, the data section at general.alignment, default 32). */
#ifndef C0VEN_GGUF_H
#define C0VEN_GGUF_H

#include <stdint.h>

#include "c0ven_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct c0ven_gguf c0ven_gguf;

/* A tensor of the file (GgufTensor, gguf.h:14-26): shape in ggml order (shape[0] the contiguous axis), its bytes
 * mapped read-only at data. name points into the reader and lives as long as it does. */
typedef struct {
  const char *name;
  uint32_t type;      /* ggml type id (c0ven_quant.h QT_*) */
  uint32_t n_dims;    /* 1 .. 4 */
  uint64_t shape[4];  /* unused dimensions are 1 */
  uint32_t shard;     /* index of the file that holds it */
  uint64_t offset;    /* byte offset in that file */
  uint64_t bytes;
  const uint8_t *data;
} gguf_tensor_info;

/* Opens and maps the file, and its sibling shards when the name has the split form (GgufModel::GgufModel,
 * gguf.cpp:175-190). Metadata keys of the first shard are kept; the split.* keys of the others are dropped. */
MOE_API moe_status gguf_open(const char *path, c0ven_gguf **out);
MOE_API void gguf_close(c0ven_gguf *g);
/* The last error's message on g (g may be null for gguf_open's and gguf_architecture's failures). */
MOE_API const char *gguf_last_error(const c0ven_gguf *g);

MOE_API uint32_t gguf_n_files(const c0ven_gguf *g);
MOE_API uint64_t gguf_n_tensors(const c0ven_gguf *g);
/* Tensor i in name order, or the tensor of a name (MOE_BAD_ARGUMENT when it is missing: GgufModel::find). */
MOE_API moe_status gguf_tensor_at(const c0ven_gguf *g, uint64_t i, gguf_tensor_info *out);
MOE_API moe_status gguf_find_tensor(const c0ven_gguf *g, const char *name, gguf_tensor_info *out);

/* Metadata (GgufModel::get_int / get_float / get_string / get_ints, gguf.cpp:234-266): integers (and bools) as int64,
 * numbers as double (integers widen), strings copied with a terminating zero into buf (len receives the length
 * without it; MOE_BAD_ARGUMENT when cap is too small), integer arrays into out (n receives the count; at most cap
 * are written). A missing key or one of another type is MOE_BAD_ARGUMENT. */
MOE_API int gguf_has_key(const c0ven_gguf *g, const char *key);
MOE_API moe_status gguf_get_int(const c0ven_gguf *g, const char *key, int64_t *out);
MOE_API moe_status gguf_get_float(const c0ven_gguf *g, const char *key, double *out);
MOE_API moe_status gguf_get_string(const c0ven_gguf *g, const char *key, char *buf, uint64_t cap, uint64_t *len);
MOE_API moe_status gguf_get_ints(const c0ven_gguf *g, const char *key, int64_t *out, uint64_t cap, uint64_t *n);

/* general.architecture of the file at path, read from its header alone (gguf_architecture, gguf.cpp:153-173). */
MOE_API moe_status gguf_architecture(const char *path, char *buf, uint64_t cap);

/* Gives the pages of bytes [off, off + bytes) of a tensor back to the kernel (GgufModel::release, gguf.cpp:280-287);
 * the bytes stay readable and are read from the file again when touched. */
MOE_API moe_status gguf_release(const c0ven_gguf *g, const char *name, uint64_t off, uint64_t bytes);

/* Bytes a tensor of type and element count takes (ggml_type_bytes, gguf.cpp:118-123); 0 for a type without a block
 * size here or a count that is not whole blocks. */
MOE_API uint64_t gguf_type_bytes(uint32_t type, uint64_t elements);

/* Loads block blk's MoE tensors into layer of ctx: the router blk.N.ffn_gate_inp.weight (n_embd x n_expert BF16) and
 * the shared gate row blk.N.ffn_gate_inp_shexp.weight (n_embd BF16), the routed experts blk.N.ffn_{gate,up,down}_exps
 * (n_embd x n_ff x n_expert, and n_ff x n_embd x n_expert for down: expert e is slice e) and, with a shared expert,
 * blk.N.ffn_{gate,up,down}_shexp. Each tensor's shape and type must be the context's (gate and up of one type); the
 * expert bytes are read from the mapping and repacked (moe_load_router / moe_load_expert). The router bias is left
 * off (the file has none). ctx's errors land in moe_last_error(ctx). */
MOE_API moe_status moe_load_layer_gguf(moe_ctx *ctx, uint32_t layer, const c0ven_gguf *g, uint32_t blk);

#ifdef __cplusplus
}
#endif

#endif
