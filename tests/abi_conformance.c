/*
 * abi_conformance.c -- replays loom's plugin loader against libloom_accel_amd.so.
 *
 * Sequence of poly/accel/plugin_linux.go:45-92 and 184-212: dlopen with
 * RTLD_NOW|RTLD_LOCAL, dlsym of all 12 v2 symbols (any missing one fails the
 * load), api_version == LOOM_ACCEL_API_VERSION, then plugin_open and, on
 * NULL, last_error(NULL).  Also checks the size contract of weight_bytes and
 * the error convention of compile_layer on bad descriptors.
 *
 * usage: abi_conformance <path-to-so> <expect_gpu:0|1>
 * Prints one line per check; exit status 0 when every check passed.
 */
#include <dlfcn.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "loom_accel.h"

static int failures = 0;

#define CHECK(cond, msg)                                   \
    do {                                                   \
        if (cond) {                                        \
            printf("ok   %s\n", msg);                      \
        } else {                                           \
            printf("FAIL %s\n", msg);                      \
            failures++;                                    \
        }                                                  \
    } while (0)

typedef int (*fn_version)(void);
typedef const char* (*fn_vendor)(void);
typedef int (*fn_npu)(void);
typedef loom_accel_plugin* (*fn_open)(const char*);
typedef void (*fn_close)(loom_accel_plugin*);
typedef size_t (*fn_wbytes)(const loom_accel_layer_desc*);
typedef int (*fn_compile)(loom_accel_plugin*, const loom_accel_layer_desc*, const void*, size_t,
                          loom_accel_compiled_layer**, double*, char*, size_t);
typedef void (*fn_release)(loom_accel_compiled_layer*);
typedef int (*fn_io)(loom_accel_compiled_layer*, size_t*, size_t*, char*, size_t);
typedef int (*fn_first)(loom_accel_compiled_layer*, double*, char*, size_t);
typedef int (*fn_infer)(loom_accel_compiled_layer*, const void*, size_t, void*, size_t, double*,
                        char*, size_t);
typedef const char* (*fn_lasterr)(loom_accel_plugin*);

int main(int argc, char** argv) {
    if (argc < 3) {
        fprintf(stderr, "usage: %s <so> <expect_gpu>\n", argv[0]);
        return 2;
    }
    const int expect_gpu = atoi(argv[2]);
    void* h = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
    if (!h) {
        printf("FAIL dlopen: %s\n", dlerror());
        return 1;
    }
    static const char* names[12] = {
        "loom_accel_api_version", "loom_accel_vendor_id",     "loom_accel_npu_available",
        "loom_accel_plugin_open", "loom_accel_plugin_close",  "loom_accel_weight_bytes",
        "loom_accel_compile_layer", "loom_accel_release_layer", "loom_accel_layer_io_bytes",
        "loom_accel_first_infer", "loom_accel_infer",         "loom_accel_last_error"};
    void* sym[12];
    int missing = 0;
    for (int i = 0; i < 12; i++) {
        sym[i] = dlsym(h, names[i]);
        if (!sym[i]) {
            printf("FAIL dlsym %s\n", names[i]);
            missing++;
        }
    }
    CHECK(missing == 0, "all 12 v2 symbols resolve");
    if (missing) return 1;
    fn_version api_version = (fn_version)sym[0];
    fn_vendor vendor_id = (fn_vendor)sym[1];
    fn_npu npu_available = (fn_npu)sym[2];
    fn_open plugin_open = (fn_open)sym[3];
    fn_close plugin_close = (fn_close)sym[4];
    fn_wbytes weight_bytes = (fn_wbytes)sym[5];
    fn_compile compile_layer = (fn_compile)sym[6];
    fn_release release_layer = (fn_release)sym[7];
    fn_io io_bytes = (fn_io)sym[8];
    fn_lasterr last_error = (fn_lasterr)sym[11];

    CHECK(api_version() == LOOM_ACCEL_API_VERSION, "api_version == 2");
    CHECK(strcmp(vendor_id(), "amd") == 0, "vendor_id == amd");
    CHECK(npu_available() == expect_gpu, "npu_available matches the machine");

    loom_accel_plugin* cpu = plugin_open("CPU");
    CHECK(cpu == NULL, "open(CPU) is refused (no CPU device in the GPU plugin)");
    CHECK(strstr(last_error(NULL), "CPU") != NULL, "last_error(NULL) explains the CPU refusal");
    CHECK(plugin_open(NULL) == NULL, "open(NULL) fails");
    CHECK(plugin_open("NPU") == NULL && strstr(last_error(NULL), "unknown device") != NULL,
          "open(unknown) fails with a message");

    loom_accel_layer_desc lin = {"BitNetLinear", "TERNARY", "m=1,k=2560,n=6912"};
    CHECK(weight_bytes(&lin) == 24 + (size_t)6912 * 160 * 4, "weight_bytes(BitNetLinear 2560->6912)");
    loom_accel_layer_desc swi = {"BitNetSwiGLU", "TERNARY", "m=8,k=2560,n=6912,eps=1e-5"};
    CHECK(weight_bytes(&swi) == 2 * (24 + (size_t)6912 * 160 * 4) + (24 + (size_t)2560 * 432 * 4) +
                                    (size_t)6912 * 4,
          "weight_bytes(BitNetSwiGLU 2560/6912)");
    loom_accel_layer_desc bad1 = {"Dense", "TERNARY", "m=1,k=4,n=4"};
    loom_accel_layer_desc bad2 = {"BitNetLinear", "FP32", "m=1,k=4,n=4"};
    loom_accel_layer_desc bad3 = {"BitNetLinear", "TERNARY", "small"};
    loom_accel_layer_desc bad4 = {"BitNetLinear", "TERNARY", "m=1,k=4"};
    CHECK(weight_bytes(&bad1) == 0 && weight_bytes(&bad2) == 0 && weight_bytes(&bad3) == 0 &&
              weight_bytes(&bad4) == 0 && weight_bytes(NULL) == 0,
          "weight_bytes == 0 for unknown layer / dtype / size");

    loom_accel_plugin* gpu = plugin_open("GPU");
    if (!expect_gpu) {
        CHECK(gpu == NULL, "open(GPU) fails without a gfx950 device");
        CHECK(strstr(last_error(NULL), "gfx950") != NULL, "last_error(NULL) names gfx950");
    } else {
        CHECK(gpu != NULL, "open(GPU) succeeds on a gfx950 box");
        if (gpu) {
            char err[512];
            loom_accel_compiled_layer* out = (loom_accel_compiled_layer*)0x1;
            int rc = compile_layer(gpu, &bad1, "", 0, &out, NULL, err, sizeof err);
            CHECK(rc == -1 && out == NULL && strstr(err, "unknown layer") != NULL,
                  "compile(unknown layer) -> -1, *out = NULL, message");
            unsigned char tiny[24 + 4] = {0};
            loom_accel_layer_desc d = {"BitNetLinear", "TERNARY", "m=1,k=4,n=1"};
            tiny[0] = 1;  /* rows */
            tiny[4] = 4;  /* cols */
            tiny[16] = 1; /* rowWords */
            tiny[20] = 1; /* nWords */
            rc = compile_layer(gpu, &d, tiny, sizeof tiny, &out, NULL, err, sizeof err);
            CHECK(rc == 0 && out != NULL, "compile(1x4 blob) succeeds");
            size_t ib = 0, ob = 0;
            CHECK(io_bytes(out, &ib, &ob, err, sizeof err) == 0 && ib == 16 && ob == 4,
                  "io_bytes = 16 / 4");
            fn_infer infer = (fn_infer)sym[10];
            float in[4] = {1, 2, 3, 4}, o[1];
            rc = infer(out, in, 12, o, 4, NULL, err, sizeof err);
            CHECK(rc == -1 && strstr(err, "input byte size mismatch") != NULL,
                  "infer with a wrong size -> -1");
            release_layer(out);
            release_layer(NULL);
            plugin_close(gpu);
        }
    }
    dlclose(h);
    printf("%d failure(s)\n", failures);
    return failures ? 1 : 0;
}
