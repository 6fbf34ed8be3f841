/*
 * ggml-mi355.h -- ggml backend for AMD MI355X (gfx950) quantized MUL_MAT.
 *
 * A ggml backend (ggml_backend_reg / ggml_backend_device / buffer type / buffer /
 * ggml_backend_i) whose supports_op claims GGML_OP_MUL_MAT on Q8_0, Q4_K, Q6_K
 * and F16 weights with F32 activations; every other op stays on the CPU backend
 * through ggml_backend_sched, the reference's own fallback contract.  It plugs in
 * where CrispEmbed picks a GPU backend: crispasr_init_gpu_backend() prefix-matches
 * the --gpu-backend string against registered device names
 * (src/core/gpu_backend_pref.h:117-152), so "mi355" selects device "MI355X0".
 * CrispEmbed never loads backends dynamically, so the host registers this one
 * once before the first crispembed_init (one line next to
 * crispembed_set_gpu_backend, src/crispembed.cpp:2802-2804):
 *     ggml_backend_register(ggml_backend_mi355_reg());
 *
 * Weights: ggml_backend_tensor_set uploads GGUF bytes unchanged (as
 * core_gguf::load_weights does, src/core/gguf_loader.cpp:480); the backend then
 * builds the kernel planes after them (see mq.h, "weight images"), so
 * get_tensor returns the original bytes and partial writes rebuild only the rows
 * they touch.  The buffer type's get_alloc_size reports the enlarged size,
 * which the reference's split loader already honours (gguf_loader.cpp:535-540).
 */
#ifndef GGML_MI355_H
#define GGML_MI355_H

#include "ggml-backend.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces a backend library's registry entry point (ggml_backend_cuda_reg and
 * the like); registry name "MI355X". */
GGML_BACKEND_API ggml_backend_reg_t ggml_backend_mi355_reg(void);
/* Direct constructor for HIP device `device` (like ggml_backend_cuda_init). */
GGML_BACKEND_API ggml_backend_t ggml_backend_mi355_init(int device);
GGML_BACKEND_API bool ggml_backend_is_mi355(ggml_backend_t backend);
GGML_BACKEND_API ggml_backend_buffer_type_t ggml_backend_mi355_buffer_type(int device);
/* Number of gfx950 devices the backend exposes. */
GGML_BACKEND_API int ggml_backend_mi355_get_device_count(void);

/* Dynamic-loading entry points of a GGML_BACKEND_DL library (what ggml's
 * GGML_BACKEND_DL_IMPL / GGML_BACKEND_DL_SCORE_IMPL define in every backend
 * library): ggml_backend_load(path) calls ggml_backend_init() for the registry
 * and requires api_version GGML_BACKEND_API_VERSION; ggml_backend_load_best()
 * ranks candidate libraries by ggml_backend_score() (0: cannot run on this
 * machine, here: no gfx950 device).  CrispEmbed itself never calls
 * ggml_backend_load (its backend choice is src/core/gpu_backend_pref.h:70-161),
 * so these serve ggml builds that discover backends at run time. */
GGML_BACKEND_API ggml_backend_reg_t ggml_backend_init(void);
GGML_BACKEND_API int ggml_backend_score(void);

/* Observer of the quantized activations the products read.  ggml's eval callback (the imatrix
 * collector's hook, src/imatrix.cpp:57-99, installed at src/crispembed.cpp:723,2483) sees a
 * MUL_MAT's F32 src1; on this backend every product first quantizes src1 to the weight's
 * vec_dot_type as ggml-cpu's from_float does (LEARNINGS.md:4826-4830), and this hook shows those
 * integer activations, so a caller can check them against ggml's quantization of the src1 it
 * reads.  No counterpart in ggml (the runner-level sibling is mq_decoder_set_observer).  While
 * set, before each MUL_MAT on a quantized weight reads its activation, the backend synchronizes
 * its stream and calls cb with the MUL_MAT node, the weight's mq type (MQ_TYPE_*), the product's
 * path (MQ_PATH_GEMM / MQ_PATH_GEMV), the device address and size of the quantized activation
 * in the layout mq_quantize_act_ex writes for that type and path (include/mq.h), and its rows
 * and K.  The activation is readable during the call only.  Grouped products (q|k|v, gate|up)
 * report the one activation once per member.  Decode-sized K-quant products quantize in a
 * separate launch while the observer is set (not inside their GEMV), so that every product is
 * reported; a product over batches whose strides do not continue the rows is not.  cb NULL:
 * off. */
typedef void (*ggml_backend_mi355_act_observer)(const struct ggml_tensor *node, int type, int path, const void *act,
                                                size_t act_bytes, int64_t rows, int64_t k, void *user);
GGML_BACKEND_API void ggml_backend_mi355_set_act_observer(ggml_backend_t backend, ggml_backend_mi355_act_observer cb,
                                                          void *user);

#ifdef __cplusplus
}
#endif
#endif
