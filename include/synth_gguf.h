/*
 * synth_gguf.h -- GGUF package reader and device loader of libsynth_hip.
 *
 * The reference loads a model package's tensors through ggml's gguf reader
 * (src/arch/qwen3-tts/weights.cpp:1-80 reads the metadata,
 * src/arch/qwen3-tts/catalog.cpp:77-104 resolves each tensor by name, type
 * and shape). These entry points give the lookup tables the gathers read
 * (talker.model.text_embedding.weight, talker.model.codec_embedding.weight,
 * talker.code_predictor.model.codec_embedding.<g>.weight) the same path into
 * device memory: parse the header on the host, then stream a tensor's bytes
 * straight into a caller-allocated device buffer that shp_get_rows /
 * shp_get_rows_sum read in place.
 *
 * Opening and inspecting run host code only (no HIP call). A handle is not
 * safe for concurrent use.
 */
#ifndef SYNTH_GGUF_H
#define SYNTH_GGUF_H

#include "synth_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct shp_gguf shp_gguf;

/*
 * Parses and validates a GGUF v2/v3 file (magic, version, key/value section,
 * tensor infos, alignment, every tensor inside the file): SHP_ERR_INVALID_ARG
 * for a malformed or truncated file, a duplicate key or tensor name, a
 * tensor offset not a multiple of general.alignment, a row not a whole number
 * of blocks; SHP_ERR_UNSUPPORTED for a tensor type this reader cannot size.
 */
shp_status_t shp_gguf_open(const char * path, shp_gguf ** out);
void         shp_gguf_close(shp_gguf * g);

uint32_t     shp_gguf_version(const shp_gguf * g);
int64_t      shp_gguf_tensor_count(const shp_gguf * g);
const char * shp_gguf_tensor_name(const shp_gguf * g, int64_t index); /* NULL when out of range */

/*
 * The named tensor as an shp_tensor (data NULL): type = its ggml type id,
 * ne = its dimensions (1 past n_dims), ggml's strides (nb[0] the element
 * size, or the block's bytes: 34 per Q8_0 block, 176 per Q5_K super-block). nbytes and file_offset may be NULL.
 * SHP_ERR_INVALID_ARG when the name is absent (ggml_get_tensor's NULL).
 */
shp_status_t shp_gguf_tensor_info(const shp_gguf * g,
                                  const char *     name,
                                  shp_tensor *     desc,
                                  uint64_t *       nbytes,
                                  uint64_t *       file_offset);

/* Metadata values; SHP_ERR_INVALID_ARG when absent or of another type, or a
 * string that does not fit `capacity` with its terminator. */
shp_status_t shp_gguf_kv_u32(const shp_gguf * g, const char * key, uint32_t * value);
shp_status_t shp_gguf_kv_string(const shp_gguf * g, const char * key, char * buf, size_t capacity);

/*
 * Streams the named tensor's bytes into device memory at device_dst (capacity
 * bytes available) through two pinned staging buffers, the read of one chunk
 * overlapping the host-to-device copy of the other, on `stream`; returns once
 * the copy has completed, with desc describing the device tensor (data =
 * device_dst). F32, F16, BF16, Q8_0, Q5_K and I32 tensors only (SHP_ERR_UNSUPPORTED
 * otherwise). The staging buffers (64 MiB pinned) are kept by the handle until
 * shp_gguf_close.
 */
shp_status_t shp_gguf_load_tensor(shp_gguf *   g,
                                  const char * name,
                                  void *       device_dst,
                                  size_t       capacity,
                                  shp_tensor * desc,
                                  shp_stream_t stream);

/*
 * Loads `count` named tensors in one pass, as the reference's weight loader
 * does for a whole package (src/gguf-metadata.cpp:20-46: every tensor of the
 * weights context read and uploaded in turn). Tensor i goes to
 * device_dsts[i] (capacities[i] bytes) and is described in descs[i], as
 * shp_gguf_load_tensor does. Every name, type and capacity is checked before
 * anything is read (the first failure's status is returned and nothing is
 * copied). The tensors' bytes then go through the staging buffers back to
 * back -- a chunk carries as many small tensors as fit, read by parallel
 * threads -- with one synchronisation at the end instead of one per tensor.
 * count = 0 does nothing and returns SHP_OK.
 */
shp_status_t shp_gguf_load_tensors(shp_gguf *          g,
                                   const char * const * names,
                                   int32_t              count,
                                   void * const *       device_dsts,
                                   const size_t *       capacities,
                                   shp_tensor *         descs,
                                   shp_stream_t         stream);

/*
 * The type the catalog requires of the talker half's matrix tensors -- the
 * text and codec embedding tables included -- under a quantization profile
 * (synthesize.quantization.profile): "BF16" -> BF16, "F16" -> F16,
 * "Q8_MIXED" -> Q8_0, "Q5_K_MIXED" -> Q5_K (src/arch/qwen3-tts/catalog.cpp:
 * 155-196, tools/synthesize-quantize/policy.cpp:49-98).
 * Unknown profiles give SHP_ERR_INVALID_ARG.
 */
shp_status_t shp_table_type_for_profile(const char * profile, int32_t * type);

#ifdef __cplusplus
}
#endif

#endif /* SYNTH_GGUF_H */
