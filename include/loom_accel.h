/*
 * loom_accel.h -- the vendor plugin ABI that loom's poly/accel loader binds,
 * API version 2, as exported by libloom_accel_amd.so.
 *
 * The declarations must match loom's own header field for field, because
 * poly/accel/plugin_linux.go resolves every symbol below with dlsym and
 * calls it through cgo (poly/accel/plugin_linux.go:45-92, 184-308).
 * Reference interface: poly/accel/include/loom_accel.h:11-66.
 *
 * Conventions (poly/accel/plugin_linux.go:200-300):
 *   - int-returning calls give 0 on success and -1 on failure; the message is
 *     copied, truncated and NUL-terminated, into the caller's err buffer;
 *   - loom_accel_plugin_open returns NULL on failure and the reason is then
 *     available from loom_accel_last_error(NULL);
 *   - weight bytes are borrowed for the duration of compile_layer only;
 *   - in/out buffers of infer are caller-owned host memory whose sizes must
 *     equal layer_io_bytes exactly; infer is synchronous.
 */
#ifndef LOOM_ACCEL_H
#define LOOM_ACCEL_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* loom's loader refuses any other value (poly/accel/plugin_linux.go:200-203). */
#define LOOM_ACCEL_API_VERSION 2

typedef struct loom_accel_plugin loom_accel_plugin;
typedef struct loom_accel_compiled_layer loom_accel_compiled_layer;

/* poly/accel/include/loom_accel.h:16-20.  For this plugin:
 *   layer_name  "BitNetLinear" | "BitNetSwiGLU"
 *   dtype       "TERNARY"
 *   size_label  "m=<rows>,k=<in>,n=<out>" plus optional ",act=<id>",
 *               ",eps=<float>", ",norm=strict|fast" (the ABI has no shape
 *               field, so the shape travels in the label). */
typedef struct loom_accel_layer_desc {
    const char* layer_name;
    const char* dtype;
    const char* size_label;
} loom_accel_layer_desc;

/* poly/accel/include/loom_accel.h:22 -- returns LOOM_ACCEL_API_VERSION. */
int loom_accel_api_version(void);
/* poly/accel/include/loom_accel.h:23 -- "amd". */
const char* loom_accel_vendor_id(void);
/* poly/accel/include/loom_accel.h:24 -- 1 when a gfx950 GPU is visible. */
int loom_accel_npu_available(void);

/* poly/accel/include/loom_accel.h:26-27 -- device "GPU" only. */
loom_accel_plugin* loom_accel_plugin_open(const char* device);
void loom_accel_plugin_close(loom_accel_plugin* plugin);

/* poly/accel/include/loom_accel.h:29 -- weight blob size the layer expects:
 * concatenated BITNET_TERNARY entity blobs (poly/entity_bitnet.go:38-55),
 * gate|up|down for SwiGLU, followed for SwiGLU by the optional fp32
 * inner-norm weights (n values). */
size_t loom_accel_weight_bytes(const loom_accel_layer_desc* desc);

/* poly/accel/include/loom_accel.h:31-39 */
int loom_accel_compile_layer(
    loom_accel_plugin* plugin,
    const loom_accel_layer_desc* desc,
    const void* weight_bytes,
    size_t weight_byte_len,
    loom_accel_compiled_layer** out,
    double* compile_ms,
    char* err,
    size_t err_len);

/* poly/accel/include/loom_accel.h:41 -- NULL is accepted. */
void loom_accel_release_layer(loom_accel_compiled_layer* layer);

/* poly/accel/include/loom_accel.h:43-48 -- fp32 wire: in m*k*4, out m*n*4
 * (SwiGLU: out m*k*4). */
int loom_accel_layer_io_bytes(
    loom_accel_compiled_layer* layer,
    size_t* in_bytes,
    size_t* out_bytes,
    char* err,
    size_t err_len);

/* poly/accel/include/loom_accel.h:50-54 -- one warm-up run on zeros. */
int loom_accel_first_infer(
    loom_accel_compiled_layer* layer,
    double* first_infer_ms,
    char* err,
    size_t err_len);

/* poly/accel/include/loom_accel.h:56-64 */
int loom_accel_infer(
    loom_accel_compiled_layer* layer,
    const void* in,
    size_t in_bytes,
    void* out,
    size_t out_bytes,
    double* infer_ms,
    char* err,
    size_t err_len);

/* poly/accel/include/loom_accel.h:66 -- NULL plugin: last open() failure. */
const char* loom_accel_last_error(loom_accel_plugin* plugin);

#ifdef __cplusplus
}
#endif

#endif /* LOOM_ACCEL_H */
