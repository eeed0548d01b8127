// The fused four-direction SRNL operator for callers that cannot allocate device memory:
// code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
//
// vh_srnl_spatial_forward takes a caller workspace for the scan's chunk-start content
// memories ([lines, chunks, d, d] fp32, written by the scan and read by the readout).  This
// variant keeps that buffer in a file-scope device array instead, so a call allocates
// nothing.  The array lives in this file's code object, which the HIP runtime loads at the
// first use of one of its kernels or symbols: only a process that calls this entry point
// holds it, and then holds kScratchBytes on every GPU it calls it on until the process ends
// (measured on MI355X in a fresh process: an ordinary SRNL call of the library adds 4 MiB of
// device memory, the first call of this entry 98 MiB; tests/test_zz_no_alloc.py checks it).
//
// The device address of the array is looked up once per device (on the entry point's first
// call with that device current) with hipGetSymbolAddress and kept; kernels receive that
// address.  Every call on a GPU uses the same array: calls that overlap on one GPU (two
// streams, two host threads) race on it.  The scan writes the state of every chunk that the
// readout reads, so nothing has to be cleared between calls.
#include <algorithm>
#include <mutex>

#include "vh_common.h"

namespace vh {
namespace {

// 96 MiB: the operator workloads of the reference's configurations fit (config 3, B = 32 at
// 56^2 with 3 heads of 32: 88.1 MB; every Tiny stage at B = 128: 58.7 MB; Base at 512^2,
// B = 8: 12.6 MB per stage).
constexpr size_t kScratchBytes = size_t(96) << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on first use).
int scratch_address(void** out) {
    int dev = -1;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(VH_ERR_LAUNCH, "hipGetDevice failed: %s", hipGetErrorString(e));
    VH_REQUIRE(dev >= 0 && dev < kMaxDevices, VH_ERR_ARG, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t se = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (se != hipSuccess || p == nullptr)
            return set_error(VH_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                             hipGetErrorString(se));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return VH_OK;
}

}  // namespace
}  // namespace vh

using namespace vh;

extern "C" {

int vh_srnl_spatial_forward_noalloc(const void* x, const void* q, int32_t io_dtype, const float* M_m,
                                    const float* M_v, const float* M_k, const float* M_eta, const float* M_alpha,
                                    const float* d_skip, int32_t skip_per_direction, const float* dir_weight,
                                    float* out, int64_t B, int64_t H, int64_t W, int64_t C, int32_t head_dim,
                                    const int64_t chunks[4], const vh_srnl_consts* consts, void* stream) {
    int rc = check_spatial_shape(B, H, W, C, head_dim);
    if (rc) return rc;
    VH_REQUIRE(chunks != nullptr, VH_ERR_ARG, "chunk lengths must not be null");
    int64_t max_chunks = 0;
    for (int r = 0; r < 4; ++r) {
        VH_REQUIRE(chunks[r] > 0 && chunks[r] <= (int64_t)1 << 30, VH_ERR_ARG, "invalid chunk length %lld",
                   (long long)chunks[r]);
        max_chunks = std::max(max_chunks, (H * W + chunks[r] - 1) / chunks[r]);
    }
    const size_t need = vh_srnl_workspace_bytes(B * 4 * (C / head_dim), max_chunks, head_dim);
    VH_REQUIRE(need <= kScratchBytes, VH_ERR_WORKSPACE,
               "vh_srnl_spatial_forward_noalloc: this call needs %zu bytes of chunk-state scratch, more than "
               "its fixed %zu; call vh_srnl_spatial_forward with a workspace instead",
               need, kScratchBytes);
    void* ws = nullptr;
    rc = scratch_address(&ws);
    if (rc) return rc;
    return srnl_spatial_forward_ws(x, q, io_dtype, M_m, M_v, M_k, M_eta, M_alpha, d_skip, skip_per_direction,
                                   dir_weight, out, B, H, W, C, head_dim, chunks, consts, ws, kScratchBytes,
                                   static_cast<hipStream_t>(stream));
}

}  // extern "C"
