/* tfq_loader.h — loading a repacked (.gturbo) checkpoint into HBM.
 *
 * The reference streams routed experts from SSD into per-layer caches and
 * mmaps the resident tensors (S/Runtime/Inference/ModelExpertIO.swift,
 * S/Infrastructure/ModelIO/ResidentBuffer.swift). Here every layer's experts
 * live in one device pool (tfq_expert_pool) and the resident tensors are
 * copied into device memory once; these calls read the reference's on-disk
 * format (packed_experts/layout.json + one file per layer, written by
 * Sources/TurboFieldfareRepack/Core/Format/GTurboJSON.swift:90-155) and produce
 * that form. All functions return the status codes of tfq.h; the reason of a
 * failure is tfq_last_error_message(). */
#ifndef TFQ_LOADER_H
#define TFQ_LOADER_H

#include <stddef.h>
#include <stdint.h>

#include "tfq.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Parsed packed_experts/layout.json (opaque, immutable once loaded). */
typedef struct tfq_expert_layout tfq_expert_layout;

/* PackedExpertsLayoutReader.load (S/Infrastructure/ModelIO/PackedExpertsLayout.swift:55-137)
 * on <model_dir>/packed_experts/layout.json, with its checks and messages:
 * TFQ_E_IO when the file is missing or unreadable (ModelError.missingFile),
 * TFQ_E_INVAL for a file larger than max_bytes or a malformed document
 * (ModelError.indexCorrupt: missing top-level keys, malformed layer /
 * expert / tensor entries, non-integer tensor bits, expert id or
 * physicalRank out of range, missing expert entries). max_bytes 0: the
 * reader's default cap, 16 MiB. An expert entry without "expert" takes the
 * count of entries placed so far, one without "physicalRank" its expert id. */
int tfq_expert_layout_load(const char *model_dir, uint64_t max_bytes, tfq_expert_layout **out);
void tfq_expert_layout_free(tfq_expert_layout *layout);

/* expertStride, numLayers, expertsPerLayer and the number of layer entries. */
int tfq_expert_layout_info(const tfq_expert_layout *layout, uint64_t *expert_stride, uint32_t *num_layers,
                           uint32_t *experts_per_layer, uint32_t *layer_entries);

/* PackedExpertsLayout.expert(layer:expert:) (PackedExpertsLayout.swift:45-48);
 * layer indexes the layer entries in file order. */
int tfq_expert_layout_expert(const tfq_expert_layout *layout, uint32_t layer, uint32_t expert,
                             uint32_t *physical_rank, uint64_t *offset, uint64_t *size);

/* Model.routedExpertOffsets (S/Runtime/Inference/ModelExpertIO.swift:40-61):
 * the sub-tensor offsets of expert 0 of a layer, 0 for a role the layout
 * lacks; file (may be NULL) receives the layer file's base name. */
int tfq_expert_layout_offsets(const tfq_expert_layout *layout, uint32_t layer, tfq_expert_offsets *offsets,
                              char *file, size_t file_capacity);

/* Stride and total bytes of the device pool tfq_expert_pool_load writes for
 * one layer of experts with hidden size d and intermediate size f, at the
 * widest code width of the layout's layers (so any layer fits). */
int tfq_expert_pool_bytes(const tfq_expert_layout *layout, uint32_t d, uint32_t f, uint64_t *stride,
                          uint64_t *bytes);

/* Loads layer `layer` of <model_dir>/packed_experts into `pool` (device
 * memory, pool_bytes from tfq_expert_pool_bytes): logical expert e (the
 * router's index, whatever its physical rank in the file) at pool +
 * e*stride as [gate_w up_w down_w gate_s gate_b up_s up_b down_s down_b],
 * weights 16-byte aligned (the file's blobs only guarantee 2 bytes) and
 * scales/biases converted from the file's BF16 to fp16 on `stream` by
 * tfq_convert_bf16_to_f16 (inexact_count_dev, device uint32 or NULL, counts
 * the values fp16 does not hold exactly). Checks each expert's nine
 * sub-tensors: U32 weights of logical shape [f, d] (gate, up) and [d, f]
 * (down) whose `bits` is 4 (the repacker) or 2 / 3 (TurboFieldfareRebits,
 * Sources/TurboFieldfareRebits/main.swift:418-441: rows of cols*bits/8
 * bytes), one width for the whole layer (else TFQ_E_UNSUPPORTED), BF16
 * scales/biases [rows, cols/64], extents inside the blob; TFQ_E_IO for a
 * missing or short layer file (ModelError.missingFile
 * "packed_experts/<file>"). Fills *desc, weight_bits included, for the MoE
 * calls. Reads the file on the calling thread; the copies and conversions
 * are queued on `stream`, which the call synchronises before returning. */
int tfq_expert_pool_load(tfq_ctx *ctx, void *stream, const tfq_expert_layout *layout, const char *model_dir,
                         uint32_t layer, uint32_t d, uint32_t f, void *pool, uint64_t pool_bytes,
                         tfq_expert_pool *desc, uint32_t *inexact_count_dev);

/* Copies bytes [file_offset, file_offset + size) of the file at `path` into
 * device memory `dst`: the resident tensor region of model_weights.bin,
 * which ResidentBuffer.init (S/Infrastructure/ModelIO/ResidentBuffer.swift:15-57)
 * maps instead. TFQ_E_IO when the file is missing or shorter than the range.
 * Synchronous (the copies are queued on `stream` and awaited). */
int tfq_resident_load(void *stream, const char *path, uint64_t file_offset, uint64_t size, void *dst);

#ifdef __cplusplus
}
#endif

#endif /* TFQ_LOADER_H */
