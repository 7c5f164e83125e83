// Kernels of the register-dequantizing quantized GEMM (qgemm_dma.h) for
// QK_PACK_U8 codes, one translation unit per packing so they compile in
// parallel.

#include <hip/hip_runtime.h>

#include <cstring>
#include <type_traits>

#include "gemm_common.h"
#include "qgemm_dma.h"
#include "qgemm_dma_launch.h"

QK_DEFINE_QDMA_LAUNCH(QDmaLaunchU8, QK_PACK_U8)
