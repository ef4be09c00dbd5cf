// Allocation-free MLA decode step: the split partials and the sparse gather
// rows live in a file-scope device array instead of caller-provided
// workspace, so a caller that cannot allocate device memory (code under HIP
// graph capture, tight serving loops, harnesses that forbid hipMalloc) can
// run a whole decode step with only its inputs and outputs.
//
// The array is resolved to a device address once per device (the first call
// on that device, with it current) through hipGetSymbolAddress; host code
// only ever hands that address to the kernels -- the array's name is a host
// stand-in, not a device pointer.  Every call on one device shares the
// array, so calls that overlap on one device (two streams, two threads) race
// on it.  Nothing in it needs clearing between calls: each decode writes
// every partial the combine then reads (the partials of the segments that
// num_splits counts), and the row translation writes every gather row.
#include <mutex>

#include "fa_common.h"

namespace fa {
namespace {

__device__ __attribute__((aligned(256))) unsigned char scratch[FA_MLA_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mutex;

// Device address of `scratch` on the current device (looked up once per device).
int scratch_ptr(unsigned char** out) {
  int dev = -1;
  FA_CHECK_HIP(hipGetDevice(&dev));
  FA_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "device %d outside [0, %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    FA_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    FA_CHECK_ARG(p != nullptr, "hipGetSymbolAddress returned NULL for the scratch array");
    g_scratch_ptr[dev] = p;
  }
  *out = static_cast<unsigned char*>(g_scratch_ptr[dev]);
  return FA_OK;
}

constexpr long long align256(long long x) { return (x + 255) / 256 * 256; }

}  // namespace
}  // namespace fa

extern "C" int64_t fa_mla_noalloc_scratch_bytes(const fa_mla_decode_args* a, int32_t mode) {
  if (a == nullptr || a->batch < 1 || a->s_q < 1 || a->h_q < 1 || a->num_parts < 1) return -1;
  const long long segs = static_cast<long long>(a->batch) + a->num_parts;
  const long long rows = static_cast<long long>(a->s_q) * a->h_q;
  long long n = fa::align256(segs * rows * fa::kDv * 2) + fa::align256(segs * rows * 4);
  if (mode != 0) {
    if (a->topk < 1) return -1;
    const long long topk_pad = static_cast<long long>(fa::cdiv(a->topk, fa::kPage)) * fa::kPage;
    n += fa::align256(static_cast<long long>(a->batch) * a->s_q * topk_pad * 4);
  }
  return n;
}

extern "C" int fa_mla_decode_noalloc(const fa_mla_decode_args* a, int32_t mode, void* stream) {
  FA_CHECK_ARG(a != nullptr, "args is NULL");
  FA_CHECK_ARG(mode >= 0 && mode <= 2, "mode %d is not 0 (dense), 1 (sparse bf16), 2 (sparse fp8)",
               mode);
  FA_CHECK_ARG(a->o_accum == nullptr && a->lse_accum == nullptr && a->sparse_rows == nullptr,
               "fa_mla_decode_noalloc keeps its workspace in the library: o_accum, lse_accum "
               "and sparse_rows must be NULL");
  const int64_t need = fa_mla_noalloc_scratch_bytes(a, mode);
  FA_CHECK_ARG(need > 0, "batch / s_q / h_q / num_parts / topk invalid");
  FA_CHECK_ARG(need <= FA_MLA_NOALLOC_SCRATCH_BYTES,
               "this call needs %lld bytes of workspace, more than the %lld-byte scratch of the "
               "allocation-free entry point; use fa_mla_decode_dense / _sparse with a workspace",
               static_cast<long long>(need), static_cast<long long>(FA_MLA_NOALLOC_SCRATCH_BYTES));
  unsigned char* base = nullptr;
  int rc = fa::scratch_ptr(&base);
  if (rc != FA_OK) return rc;
  const long long segs = static_cast<long long>(a->batch) + a->num_parts;
  const long long rows = static_cast<long long>(a->s_q) * a->h_q;
  fa_mla_decode_args w = *a;
  w.o_accum = base;
  w.lse_accum = reinterpret_cast<float*>(base + fa::align256(segs * rows * fa::kDv * 2));
  if (mode != 0) {
    w.sparse_rows = reinterpret_cast<int32_t*>(base + fa::align256(segs * rows * fa::kDv * 2) +
                                               fa::align256(segs * rows * 4));
    rc = fa_mla_sparse_rows(&w, stream);
    if (rc != FA_OK) return rc;
    rc = fa_mla_decode_sparse(&w, mode == 2 ? 1 : 0, stream);
  } else {
    rc = fa_mla_decode_dense(&w, stream);
  }
  if (rc != FA_OK) return rc;
  return fa_mla_combine(&w, stream);
}
