// mla_decode_ws.hip -- the dense wave-split decode kernel's instantiations
// (mla_splitkv_kernel<DT, 4, 1, 1, true, false, false>, DT = bf16 and fp16) and their
// launcher, mla::launch_ws_dense.  The kernel template is the one in mla_decode.hip; this
// translation unit exists so that the build can compile it with a machine scheduler of its own
// (LLVM's iterative ILP strategy), which that file's other kernels do not get.
#define MLA_WS_TU
#include "mla_decode.hip"
