// Standalone gfx950 code object of the build's asc2-style int8 matmul kernels
// (matmul_int8_kernel, matmul_dequant_kernel: int32 accumulators, or the fp16
// per-channel dequant of python/test/generalization/adv/test_matmul_quant.py:23-51),
// loaded with hipModuleLoad by the asc2 launch path (pyasc_amd/asc/runtime/module.py)
// as the reference loads the binary its compiler produced
// (python/asc/runtime/jit.py:158-186).  asc2_i8_{fast,checked}_{i32,f16} take one
// asc::i8::I8Args by value; asc_matmul_i8_plan fills it, with the grid and block,
// exactly as the library's asc_matmul_i8_* entries launch them.
#include "matmul_i8_kernels.h"

ASC_I8_KERNELS(extern "C", asc2_i8_)
