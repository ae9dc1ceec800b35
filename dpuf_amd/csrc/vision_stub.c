/*
 * vision_stub.c -- link stubs for the vision entry points that the reference
 * CLI calls (dpuf-cli.c:2570-2579, 2753; declared in the reference's
 * dpuf_vision.h:81-101).  Vision encoders are outside this library's path
 * (Mode 12 text decoding on the GPU); these exist so the unmodified CLI links
 * against libdpuf_amd.so.  Every one refuses: no image is loaded, a forward
 * returns -1, the free functions accept what the others returned (nothing).
 * The structures behind the pointer arguments are never touched, so they
 * appear here as opaque pointers.
 */
#include <stdint.h>
#include <stdlib.h>

#include "../../include/dpuf_kernels.h"

DPUF_EXPORT int32_t dpuf_vision_smart_resize(int32_t in_w, int32_t in_h, const void* cfg, int32_t* out_w,
                                             int32_t* out_h) {
    (void)in_w; (void)in_h; (void)cfg;
    if (out_w) *out_w = 0;
    if (out_h) *out_h = 0;
    return -1;
}

DPUF_EXPORT float* dpuf_vision_load_image(const char* image_path, const void* cfg, int32_t* out_w,
                                          int32_t* out_h) {
    (void)image_path; (void)cfg;
    if (out_w) *out_w = 0;
    if (out_h) *out_h = 0;
    return NULL;
}

DPUF_EXPORT void dpuf_vision_free_image(float* img_rgb_norm) { free(img_rgb_norm); }

DPUF_EXPORT int32_t dpuf_vision_forward(const void* vm, const float* img_rgb_norm, int32_t w, int32_t h,
                                        int32_t start_pos, void* out) {
    (void)vm; (void)img_rgb_norm; (void)w; (void)h; (void)start_pos; (void)out;
    return -1;
}

DPUF_EXPORT void dpuf_vision_free_output(void* out) { (void)out; }
