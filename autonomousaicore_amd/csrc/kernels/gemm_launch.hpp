// Launch functions of the bf16 MFMA GEMM kernels (gemm_kernels.inc), explicitly instantiated
// per operand layout and output type in gemm_{nt,nn,tn,tt}_{bf16,f32}.hip.
#pragma once

#include <hip/hip_runtime.h>

#include "common.hpp"
#include "gemm.hpp"

namespace aic::hip::gemm_impl {

constexpr int kMaxGroups = 8;  // products per grouped launch
// Waves of a 256x256 tile (plain, grouped and expert-ragged launches): eight, arranged 2 x 4,
// each 128 x 64 with 128 accumulator registers, so two waves share each SIMD and hide each
// other's waits (measured 1-13% faster than four 128 x 128 waves on the 1B shapes, the same
// results bit for bit).
constexpr int kDmaWaves256 = 8;

// Register-staged MFMA kernel (shapes the DMA kernel cannot take).
template <int BM, int BN, bool TA, bool TB, typename CT>
void launch_mfma(const GemmArgs& a, hipStream_t s);
// splits > 1: the K range is cut into `splits` equal parts (K % (64 splits) == 0), block z
// writes its fp32 partial to part + z M N (the caller reduces them).  Otherwise the low-rank
// term of `a` (if any) runs in the kernel's tail.
template <int BM, int BN, int BK, int S, bool TA, bool TB, typename CT>
void launch_dma(const GemmArgs& a, hipStream_t s, int splits = 1, float* part = nullptr);
// Up to kMaxGroups products of one configuration in one grid.
template <int BM, int BN, int BK, int S, bool TA, bool TB, typename CT>
void launch_dma_grouped(const GemmArgs* a, int n, hipStream_t s);
// The product with an INT4 B operand (GemmArgs::Bq), TB = a.transB.
template <int BM, int BN, int BK, int S, bool TB, typename CT>
void launch_dma_q4(const GemmArgs& a, hipStream_t s);
// Expert-ragged products (gemm_ragged).
template <int BM, int BN, int BK, int S, bool TA, bool TB, typename CT>
void launch_dma_ragged(const RaggedArgs& r, hipStream_t s);

}  // namespace aic::hip::gemm_impl
