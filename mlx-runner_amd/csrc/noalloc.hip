// Token selection that allocates nothing: mlxr_k_sample_noalloc.
//
// mlxr_k_sample's two kernels hand per-block partials (largest logit and its index of every
// 256-logit block) from the first to the second through a buffer the library allocates and grows,
// and read the position through a device word the library allocates. Callers that cannot allocate
// (code under stream capture, tight serving loops, harnesses that forbid hipMalloc) get the same
// kernels over a fixed file-scope device array instead, sized for vocabularies up to
// NOALLOC_MAX_V. Every call on a device shares that device's copy of the array: calls that overlap
// on one device race (the library serialises its own calls; concurrent callers on other streams
// must not overlap).
#include <mutex>

#include "kernels.h"
#include "model.h"

namespace mlxr {
namespace {

constexpr int NOALLOC_MAX_V = 262144;                       // logits per call at most
constexpr int NOALLOC_BLOCKS = NOALLOC_MAX_V / 256;         // sample_blocks partials (256 logits each)
constexpr size_t NOALLOC_POS_OFF = (size_t)NOALLOC_BLOCKS * 8;   // after bmax [blocks] f32, barg [blocks] i32
constexpr size_t NOALLOC_BYTES = NOALLOC_POS_OFF + 256;     // 8.25 KiB

static __device__ __align__(256) unsigned char scratch[NOALLOC_BYTES];

constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_noalloc_mu;
unsigned char* g_scratch[NOALLOC_MAX_DEVICES] = {};   // the array's device address, per device

// The position word is written by a one-thread kernel (no memset / copy node in a captured stream).
__global__ void noalloc_set_pos(int* p, int v) {
    if (threadIdx.x == 0 && blockIdx.x == 0) *p = v;
}

// The array's address on the current device, looked up once per device.
int scratch_ptr(unsigned char** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(MLXR_E_NO_DEVICE, std::string("hipGetDevice: ") + hipGetErrorString(e));
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return set_error(MLXR_E_UNSUPPORTED, "device index beyond the no-allocation table");
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return set_error(MLXR_E_GPU, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        g_scratch[dev] = static_cast<unsigned char*>(p);
    }
    *out = g_scratch[dev];
    return MLXR_OK;
}

}  // namespace
}  // namespace mlxr

using namespace mlxr;

extern "C" int mlxr_k_sample_noalloc(float* logits, int V, int32_t* hist, int32_t* status, uint64_t* rng, int pos,
                                     const mlxr_sample_params* sp, void* stream) {
    if (!logits || !hist || !status || !rng || !sp || V < 1 || pos < 0) return set_error(MLXR_E_INVALID_ARG, "sample arguments");
    if (V > NOALLOC_MAX_V)
        return set_error(MLXR_E_INVALID_ARG, "mlxr_k_sample_noalloc: V = " + std::to_string(V) + " exceeds the fixed scratch (" +
                                                 std::to_string(NOALLOC_MAX_V) + " logits)");
    unsigned char* base = nullptr;
    if (int rc = scratch_ptr(&base)) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    int* dpos = reinterpret_cast<int*>(base + NOALLOC_POS_OFF);
    hipLaunchKernelGGL(noalloc_set_pos, dim3(1), dim3(64), 0, s, dpos, pos);
    SampleArgs a;
    a.logits = logits; a.V = V; a.hist = hist; a.status = status; a.rng = rng;
    a.bmax = reinterpret_cast<float*>(base);
    a.barg = reinterpret_cast<int*>(base + (size_t)NOALLOC_BLOCKS * 4);
    a.dpos = dpos;
    a.window = sp->window; a.top_k = sp->top_k; a.penalty = sp->penalty; a.temperature = sp->temperature;
    a.top_p = sp->top_p; a.min_p = sp->min_p;
    const hipError_t e = launch_sample(a, s);
    if (e != hipSuccess) return set_error(MLXR_E_GPU, hipGetErrorString(e));
    return MLXR_OK;
}
