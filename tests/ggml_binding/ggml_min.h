/*
 * ggml_min.h — the part of ggml's public header that the backend binding in
 * binding.c touches: struct ggml_tensor with ggml's field names, order and
 * array sizes (GGML_MAX_DIMS 4, GGML_MAX_OP_PARAMS 64, GGML_MAX_SRC 10,
 * GGML_MAX_NAME 64), the two tensor types and the logging macro. It stands
 * in for ggml.h (external to voxtral.cpp, fetched at configure time by its
 * CMakeLists.txt:29-39) so that the binding compiles and runs here exactly
 * as a maintainer would paste it into a ggml backend.
 */
#ifndef VXFA_GGML_MIN_H
#define VXFA_GGML_MIN_H

#include <stdint.h>
#include <stdio.h>
#include <stddef.h>

#define GGML_MAX_DIMS 4
#define GGML_MAX_OP_PARAMS 64
#define GGML_MAX_SRC 10
#define GGML_MAX_NAME 64

enum ggml_type { GGML_TYPE_F32 = 0, GGML_TYPE_F16 = 1 };
enum ggml_op { GGML_OP_NONE = 0, GGML_OP_FLASH_ATTN_EXT = 1 };   /* the value of the op is not used here */

struct ggml_backend_buffer;

struct ggml_tensor {
    enum ggml_type type;
    struct ggml_backend_buffer * buffer;
    int64_t ne[GGML_MAX_DIMS];
    size_t  nb[GGML_MAX_DIMS];
    enum ggml_op op;
    int32_t op_params[GGML_MAX_OP_PARAMS / sizeof(int32_t)];
    int32_t flags;
    struct ggml_tensor * src[GGML_MAX_SRC];
    struct ggml_tensor * view_src;
    size_t view_offs;
    void * data;
    char name[GGML_MAX_NAME];
    void * extra;
    char padding[8];
};

#define GGML_LOG_ERROR(...) fprintf(stderr, __VA_ARGS__)

#endif
