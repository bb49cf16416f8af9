/*
 * abi_conformance.c -- replays loom's plugin loader against libloom_accel_amd.so.
 *
 * Sequence of poly/accel/plugin_linux.go:45-92 and 184-212: dlopen with
 * RTLD_NOW|RTLD_LOCAL, dlsym of all 12 v2 symbols (any missing one fails the
 * load), api_version == LOOM_ACCEL_API_VERSION, then plugin_open and, on
 * NULL, last_error(NULL).  Also checks the size contract of weight_bytes and
 * the error convention of compile_layer on bad descriptors.
 *
 * With a case file (third argument, GPU boxes), it then replays the sequence
 * of the AMD Go glue's CompileLayer / Infer:
 * weight_bytes(desc) == blob length, compile_layer, layer_io_bytes,
 * first_infer (error ignored), infer, output == the expected bytes,
 * release_layer, plugin_close.  Case file: little-endian u32 length + bytes
 * for each of layer name, size label, weight blob, input, expected output.
 *
 * usage: abi_conformance <path-to-so> <expect_gpu:0|1> [case-file]
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

/* One length-prefixed field of the case file (malloc'd, NUL-terminated). */
static unsigned char* read_field(FILE* f, size_t* len) {
    unsigned char b[4];
    if (fread(b, 1, 4, f) != 4) return NULL;
    *len = (size_t)b[0] | (size_t)b[1] << 8 | (size_t)b[2] << 16 | (size_t)b[3] << 24;
    unsigned char* p = (unsigned char*)malloc(*len + 1);
    if (!p) return NULL;
    if (*len && fread(p, 1, *len, f) != *len) {
        free(p);
        return NULL;
    }
    p[*len] = 0;
    return p;
}

/* The glue's CompileLayer + Infer sequence on one layer. */
static void replay_case(void** sym, loom_accel_plugin* gpu, const char* path) {
    FILE* f = fopen(path, "rb");
    CHECK(f != NULL, "case file opens");
    if (!f) return;
    size_t ln, ll, lb, li, lo;
    unsigned char* name = read_field(f, &ln);
    unsigned char* label = read_field(f, &ll);
    unsigned char* blob = read_field(f, &lb);
    unsigned char* in = read_field(f, &li);
    unsigned char* want = read_field(f, &lo);
    fclose(f);
    CHECK(name && label && blob && in && want, "case file parses");
    if (!(name && label && blob && in && want)) return;
    loom_accel_layer_desc d = {(const char*)name, "TERNARY", (const char*)label};
    printf("     case %s %s\n", name, label);
    CHECK(((fn_wbytes)sym[5])(&d) == lb, "weight_bytes(desc) == blob length");
    char err[512] = {0};
    loom_accel_compiled_layer* layer = NULL;
    double cms = -1.0;
    int rc = ((fn_compile)sym[6])(gpu, &d, blob, lb, &layer, &cms, err, sizeof err);
    CHECK(rc == 0 && layer != NULL && cms >= 0.0, "compile_layer succeeds");
    if (rc != 0) {
        printf("     compile error: %s\n", err);
        return;
    }
    size_t ib = 0, ob = 0;
    CHECK(((fn_io)sym[8])(layer, &ib, &ob, NULL, 0) == 0 && ib == li && ob == lo,
          "layer_io_bytes matches the case");
    double fms = 0.0;
    (void)((fn_first)sym[9])(layer, &fms, NULL, 0); /* error ignored, as the glue does */
    unsigned char* got = (unsigned char*)malloc(lo);
    double ims = -1.0;
    for (int rep = 0; rep < 3; rep++) {
        memset(got, 0xff, lo);
        rc = ((fn_infer)sym[10])(layer, in, li, got, lo, &ims, err, sizeof err);
        CHECK(rc == 0 && ims >= 0.0, "infer succeeds");
        CHECK(rc == 0 && memcmp(got, want, lo) == 0, "infer output == oracle bytes");
    }
    free(got);
    ((fn_release)sym[7])(layer);
    free(name);
    free(label);
    free(blob);
    free(in);
    free(want);
}

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
            for (int c = 3; c < argc; c++) replay_case(sym, gpu, argv[c]);
            plugin_close(gpu);
        }
    }
    dlclose(h);
    printf("%d failure(s)\n", failures);
    return failures ? 1 : 0;
}
