/*
 * ghostflow.h -- GhostFlow's Tensor-level C API, served by the MI355X
 * (gfx950) backend library (libghostflow_hip.so).
 *
 * Same entry points, argument meaning, error codes and ownership rules as the
 * reference's C FFI (ghostflow-ffi/ghostflow.h, ghostflow-ffi/src/lib.rs), so
 * a C caller of that API relinks against this library without source
 * changes.  The difference is where a tensor lives: a GhostFlowTensor here
 * owns an fp32 buffer in the HBM of the device that was current when it was
 * created, and every operation runs there (hand-written HIP kernels; matmul
 * on the library's MFMA GEMM).  Host data moves only in
 * ghostflow_tensor_create (host -> device) and ghostflow_tensor_data
 * (device -> host).
 *
 * Operations are issued on the device's default stream, in call order;
 * ghostflow_tensor_data waits for them.  A tensor handle is owned by the
 * caller and released with ghostflow_tensor_free (the reference's
 * Box::into_raw / Box::from_raw pair, ghostflow-ffi/src/lib.rs:37-40,
 * :166-171).  Reshape shares the buffer of a contiguous tensor, as
 * Tensor::reshape shares its storage (ghostflow-core/src/tensor.rs:284-309);
 * the buffer is freed with its last handle.
 */
#ifndef GHOSTFLOW_H
#define GHOSTFLOW_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GHOSTFLOW_API __attribute__((visibility("default")))

/* Status of every call (ghostflow-ffi/src/lib.rs:25-35). */
typedef enum GhostFlowError {
    Success = 0,
    InvalidShape = 1,
    InvalidData = 2,
    NullPointer = 3,
    AllocationFailed = 4,
    ComputationFailed = 5,
    Unknown = 99
} GhostFlowError;

/* Opaque tensor handle (ghostflow-ffi/src/lib.rs:12-16). */
typedef struct GhostFlowTensor GhostFlowTensor;

/* ghostflow_init (lib.rs:60-64): initializes the device backend; Success
 * when a gfx950 device is usable. */
GHOSTFLOW_API enum GhostFlowError ghostflow_init(void);

/* ghostflow_version (lib.rs:66-71): a newly allocated string, released with
 * ghostflow_free_string (lib.rs:73-79). */
GHOSTFLOW_API const char *ghostflow_version(void);
GHOSTFLOW_API void ghostflow_free_string(char *s);

/* Tensor::from_slice (lib.rs:93-117, ghostflow-core/src/tensor.rs:37-61):
 * data_len must equal the product of the shape (1 for an empty shape), else
 * InvalidShape.  NULL data, shape or out: NullPointer. */
GHOSTFLOW_API enum GhostFlowError ghostflow_tensor_create(const float *data, uintptr_t data_len,
                                                          const uintptr_t *shape, uintptr_t shape_len,
                                                          GhostFlowTensor **out);

/* Tensor::zeros / Tensor::ones (lib.rs:118-164, tensor.rs:63-70). */
GHOSTFLOW_API enum GhostFlowError ghostflow_tensor_zeros(const uintptr_t *shape, uintptr_t shape_len,
                                                         GhostFlowTensor **out);
GHOSTFLOW_API enum GhostFlowError ghostflow_tensor_ones(const uintptr_t *shape, uintptr_t shape_len,
                                                        GhostFlowTensor **out);

/* Releases a handle; NULL is a no-op (lib.rs:166-171). */
GHOSTFLOW_API void ghostflow_tensor_free(GhostFlowTensor *tensor);

/* Writes the dimensions to out_shape (room for all of them is the caller's
 * duty) and their count to out_ndim (lib.rs:174-193). */
GHOSTFLOW_API enum GhostFlowError ghostflow_tensor_shape(const GhostFlowTensor *tensor, uintptr_t *out_shape,
                                                         uintptr_t *out_ndim);

/* Copies every element to out_data (room for all of them is the caller's
 * duty) and the count to out_len (lib.rs:195-214); waits for the work that
 * produces the tensor. */
GHOSTFLOW_API enum GhostFlowError ghostflow_tensor_data(const GhostFlowTensor *tensor, float *out_data,
                                                        uintptr_t *out_len);

/* Element-wise a + b and a * b with the reference's broadcasting
 * (ghostflow-core/src/ops/arithmetic.rs:19-45, :123-200; lib.rs:216-274):
 * shapes aligned at the trailing dimension, a size-1 dimension stretched.
 * Incompatible shapes: ComputationFailed. */
GHOSTFLOW_API enum GhostFlowError ghostflow_tensor_add(const GhostFlowTensor *a, const GhostFlowTensor *b,
                                                       GhostFlowTensor **out);
GHOSTFLOW_API enum GhostFlowError ghostflow_tensor_mul(const GhostFlowTensor *a, const GhostFlowTensor *b,
                                                       GhostFlowTensor **out);

/* Tensor::matmul (lib.rs:276-304, ghostflow-core/src/ops/matmul.rs:13-42):
 * both operands at least 2-D with a[-1] == b[-2]; 2-D x 2-D is one GEMM,
 * otherwise the batched product over the broadcast batch dimensions with
 * operand batch i % (a's / b's batch count) (matmul.rs:122-170, :301-325).
 * Any failure: ComputationFailed. */
GHOSTFLOW_API enum GhostFlowError ghostflow_tensor_matmul(const GhostFlowTensor *a, const GhostFlowTensor *b,
                                                          GhostFlowTensor **out);

/* Tensor::reshape (lib.rs:306-332, tensor.rs:284-309): same element count,
 * else InvalidShape; the new handle shares the buffer. */
GHOSTFLOW_API enum GhostFlowError ghostflow_tensor_reshape(const GhostFlowTensor *tensor, const uintptr_t *new_shape,
                                                           uintptr_t new_shape_len, GhostFlowTensor **out);

/* The message of this thread's last failed ghostflow_* call, or "No error"
 * (the reference always returns "No error", lib.rs:334-337).  Owned by the
 * library: do not free. */
GHOSTFLOW_API const char *ghostflow_get_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* GHOSTFLOW_H */
