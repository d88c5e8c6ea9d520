/*
 * engine_stub.c - a stand-in for the reference engine's library (the pattern of reference
 * tests/generation_engine_stub.c): it defines the engine's own engine_load_quantized_ffn and
 * engine_last_error, and its loader calls this library's w4a16_load_quantized_ffn once per rank
 * (one rank here), as an engine that binds the library would. It is linked against
 * libw4a16.so and loaded RTLD_GLOBAL ahead of it, so its definitions come first in the global
 * lookup scope: if the library called either name through its PLT, the call would land here.
 * `stub_reentries` counts such calls; the loader returns -99 for one instead of recursing.
 */
#include <stdint.h>

int w4a16_load_quantized_ffn(void *store, const char *manifest_dir);

int stub_reentries = 0;
int stub_loads = 0;
static int depth = 0;

int engine_load_quantized_ffn(void *store, const char *manifest_dir) {
    if (depth > 0) {
        ++stub_reentries;
        return -99;
    }
    ++depth;
    ++stub_loads;
    const int st = w4a16_load_quantized_ffn(store, manifest_dir);
    --depth;
    return st;
}

const char *engine_last_error(void) { return "the stub engine's own error string"; }
