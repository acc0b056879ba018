// noalloc.hip - heph_fp8_linear_noalloc: heph_fp8_linear for callers that
// cannot allocate (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc). The activation codes, their scales and
// the large-M GEMM's K-split partials live in `scratch`, a file-scope
// device array of kNoallocScratchBytes that the code object carries: every
// GPU the library runs on holds its own copy from module load until the
// process ends. The entry point allocates nothing and frees nothing.
//
// The array's name is a host-side stand-in, not a device address: the
// device address of this GPU's copy comes from hipGetSymbolAddress, looked
// up once per device on the first call made with that device current, and
// only that address is ever handed to kernels.
//
// Layout of one call inside the array: codes [M, K] from offset 0, the f32
// scales [M, K / group_k] at the end (their size rounded up to 256 bytes),
// and between them, from the first 256-byte boundary past the codes, the
// K-split scratch (used when a split plan's partials fit there). Calls on
// one GPU share the array and it keeps the last call's contents:
// HEPH_FLAG_SKIP_QUANT reuses the codes and scales the previous call on this
// device left there (same M, K and group_k), as the reference's shared
// a_fp8_ws does. Calls that overlap on one GPU (other
// streams, other threads) race on the array and must be serialized by the
// caller. Nothing in it needs to start at zero: every byte a kernel reads
// is written earlier in the same call (or, with SKIP_QUANT, by the previous
// one).
#include <mutex>

#include "../../include/hephfp8.h"
#include "heph_kernels.h"

namespace heph {

int fp8_linear_impl(void* c, int c_dtype, const uint16_t* x_bf16, const uint8_t* w,
                    const float* w_scale, int w_block_n, int w_block_k, uint8_t* q_ws,
                    size_t q_ws_bytes, float* s_ws, size_t s_ws_floats, int M, int N, int K,
                    int group_k, int flags, void* stream, const uint16_t* gamma, float eps,
                    const heph_launch_overrides* ov);

}  // namespace heph

namespace {

constexpr size_t kNoallocScratchBytes = HEPH_NOALLOC_SCRATCH_BYTES;

__device__ __align__(256) uint8_t scratch[kNoallocScratchBytes];

constexpr int kMaxDevices = 64;
uint8_t* g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

size_t round256(size_t n) { return (n + 255) & ~(size_t)255; }

// This device's copy of `scratch` (looked up once per device, with the
// device current), or nullptr when the lookup fails.
uint8_t* scratch_on_current_device()
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    uint8_t* p = __atomic_load_n(&g_scratch_ptr[dev], __ATOMIC_ACQUIRE);
    if (p) return p;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    p = g_scratch_ptr[dev];
    if (!p) {
        void* addr = nullptr;
        if (hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)) != hipSuccess || !addr)
            return nullptr;
        p = static_cast<uint8_t*>(addr);
        __atomic_store_n(&g_scratch_ptr[dev], p, __ATOMIC_RELEASE);
    }
    return p;
}

}  // namespace

extern "C" {

int heph_fp8_linear_noalloc(void* c, int c_dtype, const uint16_t* x_bf16, const uint8_t* w,
                            const float* w_scale, int w_block_n, int w_block_k, int M, int N,
                            int K, int group_k, int flags, void* stream)
{
    // the size checks come first so that an oversized call fails the same
    // way with or without a device
    if (M < 1 || K < 16 || K % 16 || group_k < 1 || K % group_k) return HEPH_ERR_SHAPE;
    const size_t q_bytes = round256((size_t)M * (size_t)K);
    const size_t s_floats = (size_t)M * (size_t)(K / group_k);
    const size_t s_bytes = round256(s_floats * sizeof(float));
    if (q_bytes + s_bytes > kNoallocScratchBytes) return HEPH_ERR_SCRATCH;
    const int st = heph::check_device();
    if (st != HEPH_OK) return st;
    uint8_t* base = scratch_on_current_device();
    if (!base) return HEPH_ERR_DEVICE;
    // q_ws is the array less the scales: the dispatch takes the part past
    // the codes' 256-byte boundary as its K-split scratch.
    float* s_ws = reinterpret_cast<float*>(base + kNoallocScratchBytes - s_bytes);
    return heph::fp8_linear_impl(c, c_dtype, x_bf16, w, w_scale, w_block_n, w_block_k, base,
                                 kNoallocScratchBytes - s_bytes, s_ws, s_floats, M, N, K,
                                 group_k, flags, stream, nullptr, 0.0f, nullptr);
}

size_t heph_noalloc_scratch_bytes(void) { return kNoallocScratchBytes; }

}  // extern "C"
