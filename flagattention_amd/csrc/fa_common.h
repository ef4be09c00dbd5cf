// Shared definitions for the gfx950 MLA decode kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "flagattention_amd.h"

namespace fa {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef unsigned short ushortx8 __attribute__((ext_vector_type(8)));
typedef unsigned int uintx4 __attribute__((ext_vector_type(4)));
typedef unsigned int uintx2 __attribute__((ext_vector_type(2)));

#define FA_LDS __attribute__((address_space(3)))

constexpr int kPage = FA_MLA_PAGE_SIZE;   // 64 tokens per page / tile
constexpr int kDqk = FA_MLA_D_QK;         // 576
constexpr int kDv = FA_MLA_D_V;           // 512
constexpr int kRows = FA_MLA_ROWS_PER_TILE;  // 128 query rows per work-group
constexpr int kMdStride = FA_MLA_MD_STRIDE;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Set the thread-local error message (defined in fa_abi.hip).
int set_error(int code, const char* fmt, ...);

// Block-of-64 work-group count needed for n items.
__host__ __device__ inline int cdiv(int a, int b) { return (a + b - 1) / b; }

}  // namespace fa

#define FA_CHECK_ARG(cond, ...)                                   \
  do {                                                            \
    if (!(cond)) return ::fa::set_error(FA_ERR_INVALID_ARG, __VA_ARGS__); \
  } while (0)

#define FA_CHECK_HIP(expr)                                                   \
  do {                                                                       \
    hipError_t _e = (expr);                                                  \
    if (_e != hipSuccess)                                                    \
      return ::fa::set_error(FA_ERR_HIP, "%s failed: %s", #expr,             \
                             hipGetErrorString(_e));                         \
  } while (0)
