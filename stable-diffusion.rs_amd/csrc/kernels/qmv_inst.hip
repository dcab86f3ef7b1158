// qmv_inst.hip -- one dtype combination of the small-M kernel
// (qmv_kernel.hpp).  The build compiles this file once per combination with
// SDQ_XD / SDQ_SD / SDQ_OD set to the activation, scale and output dtype
// codes; qmv.hip dispatches to the instantiations by dtype.
#include "qmv_kernel.hpp"

#if !defined(SDQ_XD) || !defined(SDQ_SD) || !defined(SDQ_OD)
#error "qmv_inst.hip is compiled once per dtype combination with -DSDQ_XD=.. -DSDQ_SD=.. -DSDQ_OD=.."
#endif

namespace sdq {
namespace qmv_detail {
template void qmv_combo<SDQ_XD, SDQ_SD, SDQ_OD>(int, void *, const void *, int64_t, const uint32_t *,
                                                const void *, const void *, int, int, int, int,
                                                const kern::QmvPlan &, const kern::Epilogue &,
                                                hipStream_t, float *);
} // namespace qmv_detail
} // namespace sdq
