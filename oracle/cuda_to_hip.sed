# The caller-side edits that move a program written against the reference's
# CUDA build onto this library: the CUDA runtime header and the reference's
# check macro become their HIP counterparts, and CUDA runtime calls, types
# and enumerators (cudaX...) become hipX....  qwen3:: names, including
# Device::cuda(...), are the same in both builds and are not touched.
s|#include "qwen3/cuda/cuda_check.h"|#include "qwen3/hip/hip_check.h"|
s|#include <cuda_runtime_api.h>|#include <hip/hip_runtime_api.h>|
s|#include <cuda_runtime.h>|#include <hip/hip_runtime.h>|
s/QWEN3_CUDA_CHECK/QWEN3_HIP_CHECK/g
s/\bcudaPointerAttributes\b/hipPointerAttribute_t/g
s/\bcuda\([A-Z]\)/hip\1/g
