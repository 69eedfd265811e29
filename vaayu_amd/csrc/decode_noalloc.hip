// One-token decode that allocates nothing: `vaayu_decode_gate_up` + `vaayu_decode_down`
// with their intermediate h held in a file-scope device array instead of a caller buffer.
//
// For callers that cannot allocate (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc): they pass the inputs and the output only. The array
// `scratch` holds h [n_pairs, inter] in the activation dtype, at most kScratchBytes; each
// GPU the library runs on holds its own copy until the process ends. The gate/up kernel
// writes every element of h before the down kernel (same stream) reads it, so nothing in it
// needs clearing. All calls on one GPU share that GPU's array: calls that overlap (other
// streams, other threads) race on it.
#include <mutex>

#include "abi_internal.hpp"

namespace vaayu {

constexpr int64_t kScratchBytes = 4ll << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) char scratch[kScratchBytes];

// The device address of this GPU's `scratch`, looked up once per device (with that device
// current) by hipGetSymbolAddress; the array's name is only a host-side handle.
static void* g_scratch_ptr[kMaxDevices];
static std::once_flag g_scratch_once[kMaxDevices];
static hipError_t g_scratch_rc[kMaxDevices];

static int scratch_of(void** ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(-1, "no current HIP device (or more than 64)");
  std::call_once(g_scratch_once[dev], [dev] {
    g_scratch_rc[dev] = hipGetSymbolAddress(&g_scratch_ptr[dev], HIP_SYMBOL(scratch));
  });
  if (g_scratch_rc[dev] != hipSuccess || !g_scratch_ptr[dev])
    return set_error(-1, "hipGetSymbolAddress of the decode scratch failed");
  *ptr = g_scratch_ptr[dev];
  return 0;
}

}  // namespace vaayu

using namespace vaayu;

extern "C" int64_t vaayu_decode_noalloc_scratch_bytes(void) { return kScratchBytes; }

extern "C" int vaayu_decode_noalloc(const void* x, const int64_t* table,
                                    const void* routing_weights, int32_t rw_dtype, float* out,
                                    int32_t n_pairs, const vaayu_geom* geom, int32_t act,
                                    int32_t scale_dtype, int32_t w_round, void* stream) {
  clear_error();
  if (!geom) return set_error(-1, "null pointer argument");
  if (n_pairs <= 0 || geom->inter <= 0) return set_error(-1, "n_pairs / inter must be positive");
  if (act < 0 || act > 2) return set_error(-1, "activation dtype");
  const int64_t need = (int64_t)n_pairs * geom->inter * (act == 2 ? 4 : 2);
  if (need > kScratchBytes)
    return set_error(-3, "h [n_pairs, inter] exceeds the 4 MiB decode scratch: use "
                         "vaayu_decode_gate_up / vaayu_decode_down with a caller buffer");
  void* h = nullptr;
  if (int rc = scratch_of(&h)) return rc;
  if (int rc = vaayu_decode_gate_up(x, table, h, n_pairs, geom, act, scale_dtype, stream))
    return rc;
  return vaayu_decode_down(h, table, routing_weights, rw_dtype, out, n_pairs, geom, act,
                           scale_dtype, w_round, stream);
}
