// g4_noalloc.hip -- g4_attend_noalloc (include/g4.h): g4_attend for callers
// that cannot allocate device memory (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc).
//
// The attention score rows (reference order) or split-KV partials (parallel
// order) that g4_attend keeps in a buffer the library grows with hipMalloc
// live here in a fixed file-scope device array instead.  Each device the
// library runs on holds its own copy for the life of the process.  Host code
// never passes the array's name to a kernel: in host code it is only a
// stand-in for the symbol, so its device address is looked up once per device
// (hipGetSymbolAddress, with that device current) and that address is what
// the kernels receive.
//
// Nothing needs clearing between calls: the score kernels write every entry
// of a row that the softmax and value kernels read (the decode softmax also
// writes the zeros of its 64-key padding), and the split-KV partials are
// written before they are combined.  Every call on a device shares that
// device's array, so calls that overlap in time on one device race.
#include "g4_internal.h"

namespace {

constexpr size_t kScratchBytes = (size_t)G4_ATTEND_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

}  // namespace

static __device__ __align__(256) char scratch[kScratchBytes];

static void *g_scratch_ptr[kMaxDevices];

// The device address of `scratch` on the current device (looked up on the
// first call there).
static int scratch_on_current_device(void **out) {
    int device = 0;
    G4_HIP(hipGetDevice(&device));
    if (device < 0 || device >= kMaxDevices)
        return g4::set_error(G4_ERR_DEVICE, "g4_attend_noalloc: device %d beyond the %d supported", device,
                             kMaxDevices);
    if (!g_scratch_ptr[device]) {
        void *ptr = nullptr;
        G4_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        if (!ptr) return g4::set_error(G4_ERR_DEVICE, "g4_attend_noalloc: no address for the scratch array");
        g_scratch_ptr[device] = ptr;
    }
    *out = g_scratch_ptr[device];
    return G4_OK;
}

extern "C" int g4_attend_noalloc(void *stream, float *out, const float *q, const float *key_cache,
                                 const float *value_cache, int cache_len, int head_dim, int heads,
                                 int full_attention, int start_pos, size_t n) {
    int rc = g4::check_attend_args("g4_attend_noalloc", out, q, key_cache, value_cache, cache_len,
                                   head_dim, heads, full_attention, start_pos, n);
    if (rc) return rc;
    void *ptr = nullptr;
    rc = scratch_on_current_device(&ptr);
    if (rc) return rc;
    const g4::FixedScratch fixed{ptr, kScratchBytes};
    rc = g4::launch_attend((hipStream_t)stream, out, q, key_cache, value_cache, cache_len, head_dim, heads,
                           full_attention, start_pos, nullptr, n, nullptr, nullptr, &fixed);
    if (rc) return rc;
    G4_HIP(hipGetLastError());
    return G4_OK;
}
