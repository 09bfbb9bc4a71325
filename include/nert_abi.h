/*
 * Plain-C descriptions of one NERT node and its tensors.
 *
 * These mirror the reference seam types field for field so that a caller with
 * no C++ (ctypes, cgo, JNI) can describe a node and hand it to a device:
 *   nert_tensor_desc  <->  nert::TensorView  (include/nert/device.hpp:21-25)
 *   nert_attr_desc    <->  nert::Attribute   (include/nert/graph.hpp:61-76)
 *   dtype codes       <->  nert::DataType    (include/nert/graph.hpp:42-47)
 * The references are to files of olibartfast/nert.
 */
#ifndef NERT_ABI_H
#define NERT_ABI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types, numbered as nert::DataType declares them. */
enum nert_dtype {
    NERT_F32 = 0,
    NERT_I64 = 1,
    NERT_BOOL = 2, /* one byte per element, 0 or 1 */
    NERT_UNKNOWN = 3
};

/* A borrowed tensor: data pointer (host or device, per the callee), dtype and
 * `rank` dims. rank == -1 marks an omitted optional operand (the executor's
 * TensorView{} with dtype Unknown and null data). */
typedef struct nert_tensor_desc {
    void* data;
    int32_t dtype;
    int32_t rank;
    const int64_t* dims;
} nert_tensor_desc;

/* Attribute kinds, in the order of nert::Attribute's variant alternatives. */
enum nert_attr_kind {
    NERT_ATTR_INT = 0,
    NERT_ATTR_FLOAT = 1,
    NERT_ATTR_STRING = 2,
    NERT_ATTR_INTS = 3,
    NERT_ATTR_FLOATS = 4,
    NERT_ATTR_BOOL = 5
};

typedef struct nert_attr_desc {
    const char* name;
    int32_t kind;
    int32_t _pad;
    int64_t i;             /* INT, and BOOL (0/1) */
    float f;               /* FLOAT */
    int32_t _pad2;
    const char* s;         /* STRING (NUL-terminated) */
    const int64_t* ints;   /* INTS */
    const float* floats;   /* FLOATS */
    int64_t count;         /* element count of INTS / FLOATS */
} nert_attr_desc;

/* Status codes returned by node-level entry points. */
enum nert_status {
    NERT_OK = 0,
    NERT_INFERENCE_ERROR = 1, /* the row threw nert::InferenceException */
    NERT_OTHER_ERROR = 2,     /* any other failure (unknown op, runtime error) */
    NERT_NO_KERNEL = 3        /* the device's table has no row for op_type */
};

#ifdef __cplusplus
}
#endif

#endif /* NERT_ABI_H */
