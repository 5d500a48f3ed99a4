/*
 * Filters of the cuVS C API (cuvs/neighbors/common.h): a filter is the address of a DLManagedTensor
 * of uint32 bitset words and its kind.
 */
#pragma once

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum cuvsFilterType {
  /** Every vector is a candidate. */
  NO_FILTER = 0,
  /** One bit per id (bit j of word i is id 32 i + j); a cleared bit excludes the id. */
  BITSET = 1,
  /** One row of id bits per query, rows packed back to back. */
  BITMAP = 2
};

typedef struct {
  uintptr_t addr;
  enum cuvsFilterType type;
} cuvsFilter;

#ifdef __cplusplus
}
#endif
