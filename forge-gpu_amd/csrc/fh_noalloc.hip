// fh_noalloc.hip -- fh_sort_pairs for callers that cannot allocate device memory (code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in
// the reference.
//
// The sort's scratch (control words, look-back words, per-workgroup histogram rows and the two
// ping-pong key/value buffers) lives in one file-scope device array, `scratch`, sized for at
// most kNoAllocMaxN pairs.  Each GPU holds its own copy of the array at its own address for
// the life of the process.  The host never passes the array's name to a kernel (on the host
// it is a stand-in, not a device address): the first call on a device resolves the address
// with hipGetSymbolAddress, with that device current, and keeps it per device; every later
// launch takes that pointer.  A call builds a context on the stack whose scratch pointers
// point into the array and runs the same kernels as fh_sort_pairs on the caller's stream; it
// calls no hipMalloc, hipFree or allocating routine.  Every call on one GPU shares the array
// and finds the last call's contents: the histogram kernel that starts each sort clears what
// the sort needs cleared (histograms, tile counters, the coming passes' look-back words), so
// calls that follow one another on a stream need nothing else, while calls that overlap on
// one GPU (different streams, or threads) race on the array and must not be issued.
#include <mutex>
#include <stddef.h>
#include <stdlib.h>
#include <string.h>

#include "fh_internal.hpp"

using namespace fh;

namespace {

constexpr uint32_t kNoAllocMaxN = FH_NOALLOC_MAX_N;
constexpr size_t kAlign = 256;
constexpr size_t round_up(size_t b) { return (b + kAlign - 1) / kAlign * kAlign; }
// Layout of the array, in bytes.  The passes of a sort below kSortLargeN keys use tiles of
// kSortTile keys; the histogram kernel writes at most ceil(n / kHistChunk) rows.
constexpr size_t kTiles = (kNoAllocMaxN + kSortTile - 1) / kSortTile;
constexpr size_t kHistRows = (kNoAllocMaxN + kHistChunk - 1) / kHistChunk;
constexpr size_t kCtlBytes = 16384;  // a fixed reservation for the control block
static_assert(sizeof(Control) <= kCtlBytes, "control block exceeds its reservation");
constexpr size_t kOffCtl = 0;
constexpr size_t kOffLb = kOffCtl + kCtlBytes;
constexpr size_t kOffHist = kOffLb + round_up(kTiles * kDigitSlots * 4u);
constexpr size_t kOffKa = kOffHist + round_up(kHistRows * kDigitSlots * 4u);
constexpr size_t kBuf = round_up((size_t)kNoAllocMaxN * 4u);
constexpr size_t kOffVa = kOffKa + kBuf;
constexpr size_t kOffKb = kOffVa + kBuf;
constexpr size_t kOffVb = kOffKb + kBuf;
constexpr size_t kScratchBytes = kOffVb + kBuf;
static_assert(kNoAllocMaxN < kSortLargeN, "the no-alloc sort uses the small-tile passes only");
static_assert(kHistRows <= (size_t)kHistBlocks, "histogram rows exceed the kernel's grid cap");
static_assert(kScratchBytes == (size_t)FH_NOALLOC_SCRATCH_BYTES,
              "include/forge_hip.h states the scratch size");

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
unsigned char* g_base[kMaxDevices];  // device address of `scratch` on each device, once known
bool g_gfx950[kMaxDevices];

}  // namespace

// Address of this device's copy of `scratch` (device `dev` current), resolved once.  The
// FH_DEBUG_SPIN_LIMIT environment variable (diagnostics and tests only) sets the look-back
// poll limit of the sorts on this device at that point, like FH_OPT_SPIN_LIMIT for a context.
static int scratch_of(int dev, unsigned char** base) {
    if (dev < 0 || dev >= kMaxDevices) return FH_ENODEV;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_base[dev]) {
        hipDeviceProp_t prop;
        hipError_t e = hipGetDeviceProperties(&prop, dev);
        if (e != hipSuccess) return (int)e;
        g_gfx950[dev] = strncmp(prop.gcnArchName, "gfx950", 6) == 0;
        if (!g_gfx950[dev]) return FH_ENODEV;
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!p) return (int)hipErrorInvalidSymbol;
        if (const char* lim = getenv("FH_DEBUG_SPIN_LIMIT")) {
            const uint32_t v = (uint32_t)strtoul(lim, nullptr, 10);
            e = hipMemcpy((unsigned char*)p + kOffCtl + offsetof(Control, spin_limit), &v,
                          sizeof(v), hipMemcpyHostToDevice);
            if (e != hipSuccess) return (int)e;
        }
        g_base[dev] = (unsigned char*)p;
    }
    *base = g_base[dev];
    return FH_OK;
}

extern "C" int fh_sort_pairs_noalloc(void* stream, uint32_t* keys, uint32_t* vals, uint32_t n,
                                     uint32_t num_bits) {
    if (n && (!keys || !vals)) return set_error(FH_EINVAL, "fh_sort_pairs_noalloc: null keys or values");
    if (num_bits < 1 || num_bits > 32)
        return set_error(FH_EINVAL, "fh_sort_pairs_noalloc: num_bits=%u outside 1..32", num_bits);
    if (n > kNoAllocMaxN)
        return set_error(FH_ERANGE, "fh_sort_pairs_noalloc: n=%u exceeds the fixed scratch's %u pairs",
                         n, kNoAllocMaxN);
    if (n < 2) return FH_OK;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error((int)e, "fh_sort_pairs_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    unsigned char* base = nullptr;
    const int rc = scratch_of(dev, &base);
    if (rc)
        return set_error(rc, "fh_sort_pairs_noalloc: no gfx950 scratch on device %d (status %d)",
                         dev, rc);
    // A context on the stack over the array: only the fields the sort's launchers read.
    fh_ctx c;
    memset(&c, 0, sizeof(c));
    c.device = dev;
    c.stream = (hipStream_t)stream;
    c.max_n = kNoAllocMaxN;
    c.max_sort_tiles = (uint32_t)kTiles;
    c.ctl = (Control*)(base + kOffCtl);
    c.sort_lb = (uint32_t*)(base + kOffLb);
    c.hist_part = (uint32_t*)(base + kOffHist);
    c.ka = (uint32_t*)(base + kOffKa);
    c.va = (uint32_t*)(base + kOffVa);
    c.kb = (uint32_t*)(base + kOffKb);
    c.vb = (uint32_t*)(base + kOffVb);
    e = launch_hist_keys(&c, keys, n, num_bits, true);
    if (e == hipSuccess) e = launch_sort_passes(&c, keys, vals, keys, vals, n, num_bits);
    if (e != hipSuccess)
        return set_error((int)e, "fh_sort_pairs_noalloc: %s (%d)", hipGetErrorString(e), (int)e);
    return FH_OK;
}

// The device error flag of this device's fixed scratch (raised by a look-back that gave up):
// read after the caller's stream drains, then cleared, so each failure is reported once.
extern "C" int fh_noalloc_status(void* stream) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error((int)e, "fh_noalloc_status: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return set_error(FH_ENODEV, "fh_noalloc_status: device %d", dev);
    unsigned char* base;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        base = g_base[dev];
    }
    if (!base) return FH_OK;  // no no-alloc sort has run on this device
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing((hipStream_t)stream, &cs);
    if (e == hipSuccess && cs != hipStreamCaptureStatusNone)
        return set_error(FH_ESTATE, "fh_noalloc_status: the stream is being captured");
    e = hipStreamSynchronize((hipStream_t)stream);
    if (e != hipSuccess) return set_error((int)e, "fh_noalloc_status: %s", hipGetErrorString(e));
    unsigned char* flag = base + kOffCtl + offsetof(Control, error);
    uint32_t word = 0;
    e = hipMemcpy(&word, flag, sizeof(word), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return set_error((int)e, "fh_noalloc_status: %s", hipGetErrorString(e));
    if (!word) return FH_OK;
    const uint32_t zero = 0;
    e = hipMemcpy(flag, &zero, sizeof(zero), hipMemcpyHostToDevice);
    if (e != hipSuccess) return set_error((int)e, "fh_noalloc_status: %s", hipGetErrorString(e));
    return set_error(FH_ESTATE, "fh_noalloc_status: a no-alloc sort on device %d gave up in its "
                     "look-back (code %u); its output is wrong", dev, word);
}
