// gdn2_chunk_fwd_static: the chunkwise forward for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops, harnesses
// that forbid hipMalloc).  It is gdn2_chunk_fwd with the workspace argument
// replaced by a file-scope device array, so the call allocates nothing.
//
// The array holds the per-(chunk, head) blobs that the prep kernel writes and
// the scan kernel reads.  Prep writes every byte of each blob of the current
// call before the scan reads it, so the contents a previous call left behind
// need no clearing.  Every call on one GPU shares that GPU's array: calls that
// overlap on one GPU (two streams, or two host threads) race on it.

#include <mutex>

#include "gdn2_hip.h"
#include "gdn2_internal.h"

namespace {

constexpr int kMaxDevices = 64;

std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];  // per device: the address of `scratch` there

}  // namespace

// One copy per GPU, allocated with the code object and held until the process
// ends.  In host code this name is a host-side stand-in, not a device address:
// the host reads each device's address through hipGetSymbolAddress once, with
// that device current, and uses only that address afterwards.
static __device__ __align__(256) unsigned char scratch[GDN2_STATIC_SCRATCH_BYTES];

// Device address of `scratch` on the current device; the stream must belong to it.
static int scratch_for_stream(hipStream_t stream, void **out)
{
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return GDN2_ERR_LAUNCH;
    if (stream) {
        hipDevice_t sdev = -1;
        if (hipStreamGetDevice(stream, &sdev) != hipSuccess) return GDN2_ERR_INVALID;
        if (sdev != cur) return GDN2_ERR_INVALID;  // the kernels would get another GPU's address
    }
    if (cur < 0 || cur >= kMaxDevices) return GDN2_ERR_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[cur]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return GDN2_ERR_LAUNCH;
        g_scratch_ptr[cur] = p;
    }
    *out = g_scratch_ptr[cur];
    return GDN2_OK;
}

extern "C" int gdn2_chunk_fwd_static(const void *q, const void *k, const void *v, const void *g,
                                     const void *b, const void *w, int io_dtype, int g_dtype,
                                     void *o, const float *initial_state, float *final_state,
                                     const float *A_log, const float *dt_bias, float lower_bound,
                                     const int64_t *cu_seqlens, const int64_t *cu_seqlens_host,
                                     int num_seqs, int B, int T, int H, int K, int V, float scale,
                                     unsigned flags, void *stream)
{
    // The training workspace must outlive the call (the backward reads it): not here.
    if (flags & GDN2_FLAG_SAVE_FOR_BWD) return GDN2_ERR_INVALID;
    if (B < 0 || T < 0 || H <= 0 || K <= 0 || V <= 0) return GDN2_ERR_INVALID;
    if (cu_seqlens_host && (B != 1 || num_seqs < 0)) return GDN2_ERR_INVALID;
    const size_t need = gdn2_chunk_fwd_workspace_size(B, T, H, K, V, io_dtype, cu_seqlens_host,
                                                      num_seqs);
    if (need > static_cast<size_t>(GDN2_STATIC_SCRATCH_BYTES)) return GDN2_ERR_SCRATCH;
    void *ws = nullptr;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const int st = scratch_for_stream(s, &ws);
    if (st != GDN2_OK) return st;
    return gdn2_chunk_fwd(q, k, v, g, b, w, io_dtype, g_dtype, o, initial_state, final_state,
                          A_log, dt_bias, lower_bound, cu_seqlens, cu_seqlens_host, num_seqs, B, T,
                          H, K, V, scale, flags, ws, static_cast<size_t>(GDN2_STATIC_SCRATCH_BYTES),
                          stream);
}
