// qmm_inst.hip -- one dtype combination of the large-M tile kernel
// (qmm_kernel.hpp).  The build compiles this file once per combination with
// SDQ_XD / SDQ_SD / SDQ_OD set to the activation, scale and output dtype
// codes; qmm.hip dispatches to the instantiations by dtype.
#include "qmm_kernel.hpp"

#if !defined(SDQ_XD) || !defined(SDQ_SD) || !defined(SDQ_OD)
#error "qmm_inst.hip is compiled once per dtype combination with -DSDQ_XD=.. -DSDQ_SD=.. -DSDQ_OD=.."
#endif

namespace sdq {
namespace qmm_detail {
template void qmm_combo<SDQ_XD, SDQ_SD, SDQ_OD>(int, void *, const void *, int64_t, const uint32_t *,
                                                const void *, const void *, int, int, int, int,
                                                const kern::QmmPlan &, const kern::SplitWorkspace &,
                                                const kern::Epilogue &, hipStream_t);
} // namespace qmm_detail
} // namespace sdq
