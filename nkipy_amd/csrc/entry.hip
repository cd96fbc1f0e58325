// Compute entry points of libnkipy_hip.so (declared in include/nkipy_hip.h).
//
// The chunked causal linear-attention kernels (kernels/linattn.hip) are
// compiled into the library itself, so a caller that binds only the C ABI
// runs the scan without loading code objects or going through the traced
// plan.  Launches go to the runtime stream (nkh_init) and are asynchronous.
//
// Work split (the same arithmetic as the Python launcher): the scan is
// serial over a sequence's chunks, so with fewer than 256 sequences a
// sequence is cut into `nseg` segments run concurrently; every segment
// after the first starts from the sum of fp32 partial states over ranges
// of the earlier segments, written by nk_linattn_state_c64_d128 into a
// workspace of BH * nranges * 129 * 128 floats before the scan reads them.

#include "kernels/linattn.hip"

#include <mutex>
#include <string>

#include "../../include/nkipy_hip.h"
#include "runtime_internal.h"

namespace {

constexpr int64_t kTargetWorkgroups = 256;

struct LinAttnSplit {
  int64_t nseg, rchunks, nranges;
};

LinAttnSplit linattn_split(int64_t BH, int64_t T) {
  const int64_t nchunks = T / LC;
  int64_t nseg = 1;
  while (BH * nseg < kTargetWorkgroups && nchunks % (2 * nseg) == 0 && nchunks / (2 * nseg) >= 8) nseg *= 2;
  const int64_t cs = nchunks / nseg;
  // one range per earlier segment once that fills 3/4 of the workgroup
  // target; else halves or quarters of a segment
  const int64_t wgs = BH * (nseg - 1);
  int64_t rchunks;
  if (cs % 4 || 4 * wgs >= 3 * kTargetWorkgroups) {
    rchunks = cs;
  } else if (2 * wgs >= kTargetWorkgroups) {
    rchunks = cs / 2;
  } else {
    rchunks = cs / 4;
  }
  return {nseg, rchunks, (nseg - 1) * (cs / rchunks)};
}

int64_t workspace_bytes(int64_t BH, const LinAttnSplit &s) {
  return BH * s.nranges * (int64_t)(LD + 1) * LDV * (int64_t)sizeof(float);
}

int check_shape(int64_t BH, int64_t T) {
  if (BH <= 0 || T <= 0 || T % LC)
    return nkh_internal::set_error(NKH_ERR_INVALID, "linear attention needs BH > 0 and T a positive multiple of 64, got BH=" +
                                                        std::to_string(BH) + " T=" + std::to_string(T));
  const LinAttnSplit s = linattn_split(BH, T);
  // grid sizes, and the kernels' 32-bit byte offsets within a segment / range
  if (BH * s.nseg >= (int64_t(1) << 31) || BH * (s.nranges > 0 ? s.nranges : 1) >= (int64_t(1) << 31) ||
      (T / s.nseg) * LD * 2 >= (int64_t(1) << 31))
    return nkh_internal::set_error(NKH_ERR_INVALID, "linear attention problem too large for one launch");
  return NKH_OK;
}

int check_ptrs(const void *q, const void *k, const void *v, const void *o) {
  for (const void *p : {q, k, v, o}) {
    if (!p) return nkh_internal::set_error(NKH_ERR_INVALID, "linear attention operand is null");
    if (reinterpret_cast<uintptr_t>(p) % 16)
      return nkh_internal::set_error(NKH_ERR_INVALID, "linear attention operands must be 16-byte aligned");
  }
  return NKH_OK;
}

// Both launches on `stream`; `part` holds the partial states when the
// sequences are segmented.
int launch_linattn(const void *q, const void *k, const void *v, void *o, int64_t BH, int64_t T, float *part,
                   hipStream_t stream) {
  const LinAttnSplit s = linattn_split(BH, T);
  if (s.nranges) {
    LinAttnStateArgs sa{static_cast<const uint16_t *>(k), static_cast<const uint16_t *>(v), part, BH, T,
                        (int32_t)s.nranges, (int32_t)s.rchunks, nullptr};
    void *args[] = {&sa};
    hipError_t e = hipLaunchKernel(reinterpret_cast<const void *>(&nk_linattn_state_c64_d128),
                                   dim3((unsigned)(BH * s.nranges)), dim3(512), args, 0, stream);
    if (e != hipSuccess) return nkh_internal::hip_error(e, "launch nk_linattn_state_c64_d128");
  }
  LinAttnArgs a{static_cast<const uint16_t *>(q), static_cast<const uint16_t *>(k),
                static_cast<const uint16_t *>(v), static_cast<uint16_t *>(o),
                s.nranges ? part : nullptr, BH, T, (int32_t)s.nseg, (int32_t)s.rchunks, nullptr};
  void *args[] = {&a};
  hipError_t e = hipLaunchKernel(reinterpret_cast<const void *>(&nk_linattn_c64_d128),
                                 dim3((unsigned)(BH * s.nseg)), dim3(512), args, 0, stream);
  if (e != hipSuccess) return nkh_internal::hip_error(e, "launch nk_linattn_c64_d128");
  return NKH_OK;
}

}  // namespace

// Scratch of nkh_linear_attention_noalloc: the partial prefix states.
// Every device the library runs on holds its own copy until the process
// ends.  Host code never uses this name as an address: the per-device
// address comes from hipGetSymbolAddress at set-up (g_scratch).
static __device__ __align__(256) uint8_t scratch[NKH_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
void *g_scratch[kMaxDevices] = {};  // device address of `scratch`, per device
std::mutex g_scratch_mu;

}  // namespace

namespace nkh_internal {

// Runs in nkh_init with `device` current: look up this device's copy of
// the scratch array once.
int device_setup(int device) {
  if (device < 0 || device >= kMaxDevices)
    return set_error(NKH_ERR_INVALID, "device index " + std::to_string(device) + " beyond the supported 64");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch[device]) return NKH_OK;
  void *ptr = nullptr;
  hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return hip_error(e, "hipGetSymbolAddress(scratch)");
  if (!ptr) return set_error(NKH_ERR_HIP, "hipGetSymbolAddress(scratch) returned null");
  g_scratch[device] = ptr;
  return NKH_OK;
}

}  // namespace nkh_internal

extern "C" {

int nkh_linear_attention_workspace_size(int64_t bh, int64_t t, size_t *bytes) {
  if (!bytes) return nkh_internal::set_error(NKH_ERR_INVALID, "bytes is null");
  int rc = check_shape(bh, t);
  if (rc) return rc;
  *bytes = (size_t)workspace_bytes(bh, linattn_split(bh, t));
  return NKH_OK;
}

int nkh_linear_attention(const void *q, const void *k, const void *v, void *o, int64_t bh, int64_t t,
                         void *workspace, size_t workspace_size) {
  int rc = check_shape(bh, t);
  if (rc) return rc;
  rc = check_ptrs(q, k, v, o);
  if (rc) return rc;
  const size_t need = (size_t)workspace_bytes(bh, linattn_split(bh, t));
  if (need && (!workspace || workspace_size < need))
    return nkh_internal::set_error(NKH_ERR_INVALID, "linear attention of BH=" + std::to_string(bh) + " T=" +
                                                        std::to_string(t) + " needs a workspace of " +
                                                        std::to_string(need) + " bytes, got " +
                                                        std::to_string(workspace_size));
  if (need && reinterpret_cast<uintptr_t>(workspace) % 16)
    return nkh_internal::set_error(NKH_ERR_INVALID, "linear attention workspace must be 16-byte aligned");
  return nkh_internal::with_stream([&](hipStream_t stream, int) {
    return launch_linattn(q, k, v, o, bh, t, static_cast<float *>(workspace), stream);
  });
}

int nkh_linear_attention_noalloc(const void *q, const void *k, const void *v, void *o, int64_t bh, int64_t t) {
  int rc = check_shape(bh, t);
  if (rc) return rc;
  rc = check_ptrs(q, k, v, o);
  if (rc) return rc;
  const size_t need = (size_t)workspace_bytes(bh, linattn_split(bh, t));
  if (need > NKH_NOALLOC_SCRATCH_BYTES)
    return nkh_internal::set_error(NKH_ERR_INVALID, "linear attention of BH=" + std::to_string(bh) + " T=" +
                                                        std::to_string(t) + " needs " + std::to_string(need) +
                                                        " bytes of scratch; the no-allocation entry point "
                                                        "holds at most " +
                                                        std::to_string(NKH_NOALLOC_SCRATCH_BYTES) +
                                                        " (use nkh_linear_attention with a workspace)");
  return nkh_internal::with_stream([&](hipStream_t stream, int device) {
    void *ptr;
    {
      std::lock_guard<std::mutex> lk(g_scratch_mu);
      ptr = (device >= 0 && device < kMaxDevices) ? g_scratch[device] : nullptr;
    }
    if (!ptr) return nkh_internal::set_error(NKH_ERR_NOT_INIT, "scratch of this device is not set up");
    return launch_linattn(q, k, v, o, bh, t, static_cast<float *>(ptr), stream);
  });
}

}  // extern "C"
