/*
 * DLPack tensor interchange structures (DLPack v1.0 ABI layout).
 *
 * Only the types that the certex C API passes across its boundary are declared. The field order,
 * widths and enumerator values are those of the DLPack v1.0 specification, since callers (torch,
 * numpy, cupy, C programs) fill these structures and hand them over by pointer.
 */
#pragma once

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DLPACK_MAJOR_VERSION 1
#define DLPACK_MINOR_VERSION 0

typedef enum {
  kDLCPU         = 1,
  kDLCUDA        = 2,
  kDLCUDAHost    = 3,
  kDLOpenCL      = 4,
  kDLVulkan      = 7,
  kDLMetal       = 8,
  kDLVPI         = 9,
  kDLROCM        = 10,
  kDLROCMHost    = 11,
  kDLExtDev      = 12,
  kDLCUDAManaged = 13,
  kDLOneAPI      = 14,
  kDLWebGPU      = 15,
  kDLHexagon     = 16,
  kDLMAIA        = 17,
} DLDeviceType;

typedef struct {
  DLDeviceType device_type;
  int32_t device_id;
} DLDevice;

typedef enum {
  kDLInt          = 0U,
  kDLUInt         = 1U,
  kDLFloat        = 2U,
  kDLOpaqueHandle = 3U,
  kDLBfloat       = 4U,
  kDLComplex      = 5U,
  kDLBool         = 6U,
} DLDataTypeCode;

typedef struct {
  uint8_t code;
  uint8_t bits;
  uint16_t lanes;
} DLDataType;

typedef struct {
  void* data;
  DLDevice device;
  int32_t ndim;
  DLDataType dtype;
  int64_t* shape;
  int64_t* strides; /* NULL: compact row major */
  uint64_t byte_offset;
} DLTensor;

typedef struct DLManagedTensor {
  DLTensor dl_tensor;
  void* manager_ctx;
  void (*deleter)(struct DLManagedTensor* self);
} DLManagedTensor;

#ifdef __cplusplus
}
#endif
