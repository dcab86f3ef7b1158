// sdq_noalloc.hip -- sdq_quantized_matmul_noalloc: the raw quantized linear
// for callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc).
//
// The only scratch memory the matmul kernels use is the partial tiles of a
// split K: the large-M kernel's split-K tiles and the small-M kernel's K
// ranges (x too large for one block).  Here they live in `scratch`, a
// file-scope device
// array of kScratchFloats floats that every GPU the library runs on holds
// until the process ends.  Host code never uses the array's name as an
// address: the first call on each device takes that device's copy's address
// with hipGetSymbolAddress and keeps it.  The launch planner is told the
// array's size and does not take a split that would need more.  Calls that
// overlap on one GPU share its array and race; calls on one stream are
// ordered by it.
#include <map>
#include <mutex>

#include "kernels/launch.hpp"
#include "sdq_internal.hpp"

namespace sdq {
namespace {

constexpr size_t kScratchFloats = size_t(4) << 20; // 16 MiB per device

static __device__ __align__(256) float scratch[kScratchFloats];

// The device address of `scratch` on `device` (current), taken once.
float *scratch_for(int device) {
  static std::mutex mu;
  static std::map<int, float *> ptrs;
  std::lock_guard<std::mutex> lock(mu);
  auto it = ptrs.find(device);
  if (it != ptrs.end()) return it->second;
  void *p = nullptr;
  hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
  if (!p) fail("hipGetSymbolAddress(scratch) returned no address");
  ptrs[device] = static_cast<float *>(p);
  return static_cast<float *>(p);
}

} // namespace
} // namespace sdq

using namespace sdq;

extern "C" int sdq_quantized_matmul_noalloc(void *y, int y_dtype, const void *x, int x_dtype,
                                            int64_t ldx, const uint32_t *w, const void *scales,
                                            const void *biases, int s_dtype, int64_t M, int64_t N,
                                            int64_t K, int group_size, int bits, const void *bias,
                                            int bias_dtype, int activation, void *hip_stream) {
  SDQ_GUARD("quantized_matmul_noalloc", {
    if (M < 0 || N < 0 || K <= 0) fail("M, N must be >= 0 and K > 0");
    if (!is_float_dtype(x_dtype) || !is_float_dtype(s_dtype) || !is_float_dtype(y_dtype))
      fail("dtypes must be float32, bfloat16 or float16");
    if (bias && !is_float_dtype(bias_dtype)) fail("bias dtype must be float32, bfloat16 or float16");
    if (activation != SDQ_ACT_NONE && activation != SDQ_ACT_GELU_APPROX)
      fail("activation must be SDQ_ACT_NONE or SDQ_ACT_GELU_APPROX, got " + std::to_string(activation));
    if (group_size != 64 && group_size != 128)
      fail("the quantized matmul kernels take group size 64 or 128, got " + std::to_string(group_size));
    if (bits != 4 && bits != 8)
      fail("the quantized matmul kernels take 4 or 8 bits, got " + std::to_string(bits));
    if (K % group_size != 0) fail("K must be a multiple of group_size");
    if (M == 0 || N == 0) return 0;
    if (!y || !x || !w || !scales || !biases) fail("NULL pointer argument");
    int device = 0;
    hip_check(hipGetDevice(&device), "hipGetDevice");
    const hipStream_t stream = static_cast<hipStream_t>(hip_stream);
    kern::Epilogue ep;
    ep.bias = bias;
    ep.bias_dtype = bias ? bias_dtype : 0;
    ep.act = activation;
    if (kern::qmv_takes(M, N, K)) {
      // The small-M kernel's partial tiles (a large x cut into K ranges) go
      // to the scratch when they fit; otherwise it takes a plan without.
      kern::QmvPlan plan = kern::plan_qmv(M, N, K, group_size, bits, cu_count(device));
      if (plan.partial_floats > kScratchFloats)
        plan = kern::plan_qmv(M, N, K, group_size, bits, cu_count(device), false);
      kern::qmv(y, y_dtype, x, x_dtype, ldx, w, scales, biases, s_dtype, M, N, K, group_size, bits,
                plan, ep, stream, plan.ranges > 1 ? scratch_for(device) : nullptr);
      return 0;
    }
    // The fixed scratch takes the data-parallel plan only (no stream-K flags).
    const kern::QmmPlan plan = kern::plan_qmm(M, N, K, bits, cu_count(device), kScratchFloats, false);
    if (plan.partial_floats > kScratchFloats)
      fail("the launch needs " + std::to_string(plan.partial_floats * sizeof(float)) +
           " bytes of split-K scratch; the no-allocation entry point holds " +
           std::to_string(kScratchFloats * sizeof(float)));
    kern::SplitWorkspace ws;
    if (plan.dp_tiles < plan.tiles) ws.partial = scratch_for(device);
    kern::qmm(y, y_dtype, x, x_dtype, ldx, w, scales, biases, s_dtype, M, N, K, group_size, bits, plan,
              ws, ep, stream);
  });
}
