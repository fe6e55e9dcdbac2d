// Decode attention that allocates nothing: the split-K partials live in a file-scope device
// array instead of a caller workspace (lf_decode_attention_noalloc, include/logitfill_amd.h).
//
// ``scratch`` is one fixed-size array per GPU, created when the code object is loaded onto
// that device and held until the process ends.  In host code its name is only a stand-in for
// the device symbol, so the device address is looked up once per device with
// hipGetSymbolAddress (with that device current) and that address -- never the name -- is what
// kernels receive.  Every call on a GPU shares the GPU's array: calls that overlap on one GPU
// (different streams, host threads) race on it.  The partials need no initialisation, so
// nothing is cleared.
#include <mutex>

#include "decode_common.hpp"

namespace lf {
int32_t decode_checked(const lf_packed_layer* layer, const lf_decode_args* args, void* workspace,
                       int64_t workspace_bytes, void* stream);
}

namespace {

constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[LF_NOALLOC_SCRATCH_BYTES];

std::mutex g_scratch_lock;
void* g_scratch_ptr[kMaxDevices];  // device address of ``scratch`` per device (null: not looked up)

// Device address of this device's scratch array; 0 or a hipError_t.
int scratch_address(int device, void** out) {
    std::lock_guard<std::mutex> guard(g_scratch_lock);
    if (!g_scratch_ptr[device]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return static_cast<int>(e);
        if (!ptr) return static_cast<int>(hipErrorInvalidSymbol);
        g_scratch_ptr[device] = ptr;
    }
    *out = g_scratch_ptr[device];
    return LF_OK;
}

}  // namespace

extern "C" {

int32_t lf_decode_attention_noalloc(const lf_packed_layer* layer, const lf_decode_args* args, void* stream) {
    if (!layer) return LF_E_NULL;
    if (!args) return lf::decode_checked(layer, args, nullptr, 0, stream);  // the shared checks' verdict
    const int64_t rows = static_cast<int64_t>(args->n_q) * (args->q_len > 1 ? args->q_len : 1);
    if (args->n_q <= 0 || rows > (1 << 20) || args->n_work <= 0 || layer->head_dim <= 0) return LF_E_SHAPE;
    const int64_t need = lf_decode_workspace_bytes(static_cast<int32_t>(rows), layer->head_dim, args->n_work);
    if (need < 0) return LF_E_SHAPE;
    if (need > static_cast<int64_t>(LF_NOALLOC_SCRATCH_BYTES)) return LF_E_WORKSPACE;
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return static_cast<int>(e);
    if (device < 0 || device >= kMaxDevices) return LF_E_UNSUPPORTED;
    void* ptr = nullptr;
    const int rc = scratch_address(device, &ptr);
    if (rc != LF_OK) return rc;
    return lf::decode_checked(layer, args, ptr, static_cast<int64_t>(LF_NOALLOC_SCRATCH_BYTES), stream);
}

int64_t lf_noalloc_scratch_bytes(void) { return static_cast<int64_t>(LF_NOALLOC_SCRATCH_BYTES); }

}  // extern "C"
