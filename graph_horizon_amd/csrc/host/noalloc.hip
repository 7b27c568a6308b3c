// gh_attention_decode_noalloc: decode attention for callers that cannot allocate device memory
// (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc). It runs the
// kernels of gh_attention_decode, with the split partials and merge counters in a file-scope
// device array of fixed size instead of the backend's growable workspace, and allocates
// nothing (no hipMalloc, hipFree or allocating library call).
//
// The array is one per GPU the library runs on (each device holds its own copy until the
// process ends). Host code never passes the array's name to a kernel — in host code it is only
// a stand-in symbol; gh_create resolves this device's address with hipGetSymbolAddress, with
// the device current, and every use goes through that address.
//
// Every call on a GPU shares that GPU's array and finds what the last call left: the merge
// counters, which must start at zero, are cleared by a fill kernel at the start of each call
// (and every launch leaves them zero again). Calls that overlap on one GPU (other streams,
// other backends on the same device) race on the array.
#include <hip/hip_runtime.h>

#include "internal.h"

namespace {
// Layout: merge counters (u32, one per kv head) in the first kNoAllocCounterBytes, then the
// split partials (m, l, acc[128] per (query head, split)).
constexpr size_t kNoAllocScratchBytes = (size_t)1 << 20;
constexpr size_t kNoAllocCounterBytes = 4096;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
}  // namespace

namespace gh {
int noalloc_init(gh_backend* b) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
        return fail(b, GH_E_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    b->noalloc_scratch = ptr;
    return GH_OK;
}
}  // namespace gh

using namespace gh;

extern "C" int gh_attention_decode_noalloc(gh_backend* b, gh_encoder* enc, const gh_buf* out,
                                           const gh_buf* q, const gh_kv* kv, uint32_t q_heads,
                                           uint32_t pos, uint32_t layer) {
    int rc = check_enc(b, enc);
    if (rc) return rc;
    if (!b->noalloc_scratch) return latch(enc, fail(b, GH_E_STATE, "attention_decode_noalloc: no scratch"));
    rc = check_attention(b, out, q, kv, q_heads, pos, 1, layer);
    if (rc) return latch(enc, rc);
    const size_t counters = (size_t)kv->kv_heads;
    const uint32_t splits = attention_splits(b, pos + 1, kv->kv_heads, 1);
    if (counters * 4 > kNoAllocCounterBytes ||
        attention_workspace(1, q_heads, splits) > kNoAllocScratchBytes - kNoAllocCounterBytes)
        return latch(enc, fail(b, GH_E_RANGE,
                               "attention_decode_noalloc: the heads x splits partials exceed its "
                               "1 MiB scratch (4 KiB of counters, then q_heads x splits x 520 B)"));
    char* base = (char*)b->noalloc_scratch;
    GhEltArgs clear{(uint64_t)base, 0, 0, (uint32_t)counters, 0u};
    rc = launch(b, K_FILL_U32, (uint32_t)((counters + 255) / 256), 1, 1, 256, &clear);
    if (rc) return latch(enc, rc);
    const AttnScratch s{base + kNoAllocCounterBytes, kNoAllocScratchBytes - kNoAllocCounterBytes, base,
                        kNoAllocCounterBytes / 4};
    return latch(enc, op_attention(b, out, q, kv, q_heads, pos, 1, layer, nullptr, pos, &s));
}
