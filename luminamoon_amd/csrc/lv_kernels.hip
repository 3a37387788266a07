// The kernels of one buffer mode (LV_MODE = LV_BUFFER_TDCLM, _DUAL, _T1 or _T2): every template
// instantiation of unit_kernel and fold_kernel that mode's launches can pick. The build compiles
// this file once per mode, in parallel, and links the four objects with the host side.
#include "lv_device.h"

#ifndef LV_MODE
#error "build with -DLV_MODE=<buffer mode code>"
#endif

namespace lv {

#if LV_MODE == LV_BUFFER_TDCLM
KernelFn pick_kernel_tdclm(int pt, int st, int pass, uint32_t flags, bool table) {
    return pick_param<LV_BUFFER_TDCLM>(pt, st, pass, flags, table);
}
KernelFn pick_fold_tdclm(int pass) { return pick_fold_pass<LV_BUFFER_TDCLM>(pass); }
#elif LV_MODE == LV_BUFFER_DUAL
KernelFn pick_kernel_clm(int pt, int st, int pass, uint32_t flags, bool table) {
    return pick_param<LV_BUFFER_DUAL>(pt, st, pass, flags, table);
}
KernelFn pick_fold_clm(int pass) { return pick_fold_pass<LV_BUFFER_DUAL>(pass); }
#elif LV_MODE == LV_BUFFER_T1
KernelFn pick_kernel_t1(int pt, int st, int pass, uint32_t flags, bool table) {
    return pick_param<LV_BUFFER_T1>(pt, st, pass, flags, table);
}
KernelFn pick_fold_t1(int pass) { return pick_fold_pass<LV_BUFFER_T1>(pass); }
#elif LV_MODE == LV_BUFFER_T2
KernelFn pick_kernel_t2(int pt, int st, int pass, uint32_t flags, bool table) {
    return pick_param<LV_BUFFER_T2>(pt, st, pass, flags, table);
}
KernelFn pick_fold_t2(int pass) { return pick_fold_pass<LV_BUFFER_T2>(pass); }
#else
#error "unknown LV_MODE"
#endif

}  // namespace lv
