// The unit kernels of the bench workloads, instantiated on their own so that
// tests/test_valu_budget.py can compile them to gfx950 assembly (device code only, never linked
// or run) and count the VALU instructions of their hot path: the vector path of a whole unit with
// every wave-uniform guard on its fast side.
#include "lv_device.h"

namespace lv {

// cfg5: T2, bf16 param and grad, f32 m/v (the headline step)
template __global__ void unit_kernel<LV_BUFFER_T2, LV_DTYPE_BF16, LV_DTYPE_F32, kFused,
                                     static_flags(LV_DTYPE_BF16, kFused), false>(const Args);
// cfg5 --state param: bf16 m/v
template __global__ void unit_kernel<LV_BUFFER_T2, LV_DTYPE_BF16, LV_DTYPE_BF16, kFused,
                                     static_flags(LV_DTYPE_BF16, kFused), false>(const Args);
// cfg4: T1, bf16 param and grad, f32 m
template __global__ void unit_kernel<LV_BUFFER_T1, LV_DTYPE_BF16, LV_DTYPE_F32, kFused,
                                     static_flags(LV_DTYPE_BF16, kFused), false>(const Args);
// cfg4 --state param: bf16 m
template __global__ void unit_kernel<LV_BUFFER_T1, LV_DTYPE_BF16, LV_DTYPE_BF16, kFused,
                                     static_flags(LV_DTYPE_BF16, kFused), false>(const Args);
// cfg4 --pdt f16 --state param: fp16 param and grad, m in the fp16 container as bf16 bits
template __global__ void unit_kernel<LV_BUFFER_T1, LV_DTYPE_F16, LV_DTYPE_BF16, kFused,
                                     static_flags(LV_DTYPE_F16, kFused), false>(const Args);
// cfg3: CLM, f32
template __global__ void unit_kernel<LV_BUFFER_DUAL, LV_DTYPE_F32, LV_DTYPE_F32, kFused,
                                     static_flags(LV_DTYPE_F32, kFused), false>(const Args);
// cfg2: TD-CLM, f32, table launch
template __global__ void unit_kernel<LV_BUFFER_TDCLM, LV_DTYPE_F32, LV_DTYPE_F32, kFused,
                                     static_flags(LV_DTYPE_F32, kFused), true>(const Args);

}  // namespace lv
