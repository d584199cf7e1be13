// Standalone gfx950 code object of asc2 vadd_kernel
// (python/test/asc2/kernels/test_vadd.py:16-28), loaded with hipModuleLoad by the
// asc2 launch path (pyasc_amd/asc/runtime/module.py) as the reference loads the
// binary its compiler produced (python/asc/runtime/jit.py:158-186).  The kernels
// have C names for hipModuleGetFunction; their bodies are the library's
// (vadd_kernels.h).  Arguments (natural alignment, 8-byte pointers):
//   asc2_vadd_vec_<dt>(const void* x, const void* y, void* out, int64_t n_vec)
//       16-byte vectors [0, n_vec); grid = ceil(n_vec / 1024), 256 threads
//   asc2_vadd_elem_<dt>(const void* x, const void* y, void* out, int64_t begin, int64_t end)
//       elements [begin, end), one per thread; grid = ceil((end - begin) / 256), 256 threads
// Neither kernel reads its grid size, so the launch geometry is the caller's alone.
#include "vadd_kernels.h"

using asc::vadd::kThreads;
using asc::vadd::u32x4;

#define ASC2_VADD_CODE_OBJECT_KERNELS(NAME, OP)                                                                    \
  extern "C" __global__ void __launch_bounds__(kThreads)                                                           \
      asc2_vadd_vec_##NAME(const u32x4* __restrict__ x, const u32x4* __restrict__ y, u32x4* __restrict__ out,      \
                           int64_t n_vec) {                                                                        \
    asc::vadd::vec_body<asc::vadd::OP>(x, y, out, n_vec);                                                          \
  }                                                                                                                \
  extern "C" __global__ void __launch_bounds__(kThreads)                                                           \
      asc2_vadd_elem_##NAME(const asc::vadd::OP::T* __restrict__ x, const asc::vadd::OP::T* __restrict__ y,        \
                            asc::vadd::OP::T* __restrict__ out, int64_t begin, int64_t end) {                     \
    asc::vadd::element_body<asc::vadd::OP>(x, y, out, begin, end);                                                 \
  }

ASC2_VADD_CODE_OBJECT_KERNELS(f32, AddF32)
ASC2_VADD_CODE_OBJECT_KERNELS(f16, AddF16)
ASC2_VADD_CODE_OBJECT_KERNELS(bf16, AddBF16)
ASC2_VADD_CODE_OBJECT_KERNELS(i32, AddI32)
