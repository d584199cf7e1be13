// Standalone gfx950 code object of the two asc2 softmax_kernel signatures
// (python/test/asc2/kernels/test_softmax.py:16-27, test_softmax_fused.py:16-24),
// loaded with hipModuleLoad by the asc2 launch path (pyasc_amd/asc/runtime/module.py)
// as the reference loads the binary its compiler produced
// (python/asc/runtime/jit.py:158-186).  One kernel per row body of
// softmax_kernels.h, with C names (asc2_softmax_<body>) for hipModuleGetFunction;
// every kernel takes
//   (const void* x, void* out, int64_t rows, int64_t stride, int32_t len, int32_t flag)
// and asc_softmax_plan names the kernel, grid, block and arguments of a launch,
// the same plan the library's asc_softmax_* entries launch.
#include "softmax_kernels.h"

ASC_SOFTMAX_KERNELS(extern "C", asc2_softmax_)
