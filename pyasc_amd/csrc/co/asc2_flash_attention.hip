// Standalone gfx950 code object of the build's asc2-style flash_attention_fwd_kernel,
// loaded with hipModuleLoad by the asc2 launch path (pyasc_amd/asc/runtime/module.py)
// as the reference loads the binary its compiler produced
// (python/asc/runtime/jit.py:158-186).  asc2_fa_fwd_d64 / asc2_fa_fwd_d128 take one
// asc::fa::FaArgs by value; asc_flash_attention_plan fills it, with the grid and
// block, exactly as the library's asc_flash_attention_fwd_bf16 launches them.
#include "flash_attn_kernels.h"

ASC_FA_KERNELS(extern "C", asc2_fa_fwd_)
