// Standalone gfx950 code object of the asc2 elementwise kernels beside vadd:
//   leaky_relu_kernel  python/test/asc2/kernels/test_leaky_relu.py:16-26
//   vmuladd_kernel     python/test/asc2/kernels/test_vmuladd.py:16-31
//   gelu_kernel        python/test/asc2/kernels/test_gelu.py:19-33
// loaded with hipModuleLoad by the asc2 launch path (pyasc_amd/asc/runtime/module.py)
// as the reference loads the binary its compiler produced
// (python/asc/runtime/jit.py:158-186).  The kernels have C names
// (asc2_leaky_relu_vec_f32, ...) for hipModuleGetFunction; their bodies and
// arguments are the library's (elementwise_kernels.h lists them).
#include "elementwise_kernels.h"

ASC_ELEMENTWISE_KERNELS(extern "C", asc2_)
