// Standalone gfx950 code object of the asc2 matmul kernels
// (python/test/asc2/kernels/test_matmul_{mnblock,tiled,fixpipe,l0c_to_l1}.py), loaded
// with hipModuleLoad by the asc2 launch path (pyasc_amd/asc/runtime/module.py) as the
// reference loads the binary its compiler produced (python/asc/runtime/jit.py:158-186).
// asc2_mm_<kind>_<out> take one asc::mm::GemmArgs by value; asc_matmul_plan fills it,
// with the kernel, grid and block, exactly as the library's asc_matmul launches them.
#include "matmul_kernels.h"

ASC_MM_KERNELS(extern "C", asc2_mm_)
