/* dsv4_expert_store.h — safetensors checkpoint reader that fills the
 * HBM-resident expert tensors of the routed MoE path (host code, C ABI).
 *
 * Library: dsv4-flash-gb10-runtime_amd/kernel/expert-store/libdsv4_expert_store.so
 *
 * The reference keeps routed experts in a 64-per-layer LRU hot set filled on
 * demand from CPU memory maps that a Python loader registers
 * (kernel/cpp-engine-mxfp4/hotset.cu:211-520, runtime/mxfp4_loader.py). On
 * MI355X all 43 x 256 experts (147 GB) stay resident in HBM, so the LRU
 * collapses to one load per layer into the expert-major tensors that
 * mxfp4_moe_layer / mxfp4_moe_grouped_gemv read in place:
 *   packed [n_experts, rows, cols/2], scale [n_experts, rows, cols/32].
 * Checkpoint layout (runtime/mxfp4_loader.py:35-48):
 *   layers.{L}.ffn.experts.{E}.w{1|2|3}.weight   I8       [rows, cols/2]
 *   layers.{L}.ffn.experts.{E}.w{1|2|3}.scale    F8_E8M0  [rows, cols/32]
 * A store is not thread-safe; use one per thread. All pointers named *_dev are
 * device pointers; everything else is host memory. */
#ifndef DSV4_EXPERT_STORE_H
#define DSV4_EXPERT_STORE_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct dsv4_store dsv4_store;

/* Opens a snapshot: a directory with model.safetensors.index.json and its
 * shards (the Hugging Face layout read by runtime/mxfp4_loader.py:103-122),
 * a directory with a single model.safetensors, or one .safetensors file.
 * Every shard header is parsed here. Returns NULL on error (reason on stderr). */
dsv4_store* dsv4_store_open(const char* path);

/* Closes the shard files and frees the store (NULL is accepted). Always 0. */
int dsv4_store_close(dsv4_store* store);

/* Number of tensors in the snapshot (-2 for a NULL store). */
int dsv4_store_count(const dsv4_store* store);

/* Tensor metadata: dtype string (e.g. "I8", "F8_E8M0", "BF16"; at most 15
 * characters plus NUL), up to 8 dims, byte size. Returns 0; -1 no such
 * tensor; -2 bad arguments (NULL pointers); -3 more than 8 dims. */
int dsv4_store_tensor_info(const dsv4_store* store, const char* name, char dtype[16],
                           int64_t shape[8], int* ndim, int64_t* nbytes);

/* Copies a tensor's bytes into host memory. Returns 0; -1 no such tensor;
 * -2 bad arguments; -3 capacity < the tensor's size; -5 read error. */
int dsv4_store_read(const dsv4_store* store, const char* name, void* dst, int64_t capacity);

/* Copies a tensor's bytes to device memory through a pinned staging buffer
 * (hipMemcpyAsync on `stream`); returns when the copy is complete. Returns as
 * dsv4_store_read, plus -6 for a HIP error. */
int dsv4_store_load_tensor(dsv4_store* store, const char* name, void* dst_dev, int64_t capacity,
                           hipStream_t stream);

/* Loads projection `proj` ("w1", "w2" or "w3") of layer `layer` for experts
 * 0 .. n_experts-1 into
 *   packed_dev + e * packed_expert_stride   (the .weight bytes, I8)
 *   scale_dev  + e * scale_expert_stride    (the .scale bytes, F8_E8M0)
 * Every expert must have the same shapes: weight [rows, cols/2], scale
 * [rows, cols/32]; *rows and *cols (if not NULL) receive rows and cols.
 * Shard reads overlap the host-to-device copies (two pinned buffers, copies
 * on `stream`); returns when every copy is complete. Returns 0; -1 a tensor
 * is missing; -2 bad arguments (NULL, n_experts < 1, unknown proj); -3 a
 * stride is smaller than an expert's bytes; -4 wrong dtype or shape, or
 * shapes differing between experts; -5 read error; -6 HIP error. */
int dsv4_store_load_experts(dsv4_store* store, int layer, const char* proj, int n_experts,
                            void* packed_dev, int64_t packed_expert_stride, void* scale_dev,
                            int64_t scale_expert_stride, int64_t* rows, int64_t* cols,
                            hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DSV4_EXPERT_STORE_H */
