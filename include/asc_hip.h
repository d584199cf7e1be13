/*
 * asc_hip.h -- C ABI of libasc_hip.so, the MI355X (gfx950) replacement for the
 * launch path of PyAsc's asc2 tile kernels.
 *
 * In the reference a kernel launch ends in one generic C entry point,
 *   KernelLaunchWrapper(stub, blockNum, args, argsSize, smDesc, stream)
 *   (python/asc/lib/runtime/rt_wrapper.cpp:189-193, bound by ctypes in
 *    python/asc/lib/runtime/interface.py:323-339),
 * which receives a packed little-endian argument blob built by
 * Launcher.launch_kernel (python/asc/runtime/launcher.py:156-195).
 * Here there is no JIT binary: every kernel the asc2 tutorials and tests compile
 * is a hand-written HIP kernel, so each gets a typed entry point instead of the
 * blob.  Each entry point keeps the reference kernel's argument meaning:
 * global-address buffers, runtime sizes, the tile-size ConstExprs and the
 * logical block count `grid` (the `kernel[grid]` value).  The library picks its
 * own physical HIP grid but writes exactly the elements the reference kernel
 * body would write for that logical grid.
 *
 * Conventions
 *  - Every function returns int32_t: 0 on success, a positive hipError_t value
 *    when the HIP runtime failed, or a negative ASC_ERR_* code for argument
 *    errors detected before any launch (nothing is launched then).  The
 *    reference raised RuntimeError("Function X returned N") on nonzero
 *    (python/asc/lib/runtime/state.py:63-75); the Python layer does the same.
 *  - asc_last_error() returns a thread-local description of the last failure.
 *  - All buffers are device pointers owned by the caller; the library never
 *    allocates device memory.  `stream` is a hipStream_t (NULL = legacy
 *    default stream).  Launches are asynchronous on that stream.
 *  - Sizes are int64_t, element counts (not bytes) unless stated.
 */
#ifndef ASC_HIP_H
#define ASC_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* asc_stream_t; /* hipStream_t */

/* Error codes (negative = rejected before launch). */
#define ASC_OK 0
#define ASC_ERR_INVALID_ARG (-1)
#define ASC_ERR_UNSUPPORTED (-2)
#define ASC_ERR_ALIGNMENT (-3)
#define ASC_ERR_BUSY (-4) /* a shared resource is still in use by another stream */

/* Element type codes, named after asc.language.core.dtype
 * (python/asc/language/core/dtype.py:111-124). */
#define ASC_DT_FLOAT32 0
#define ASC_DT_FLOAT16 1
#define ASC_DT_BFLOAT16 2
#define ASC_DT_INT32 3
#define ASC_DT_INT8 4
#define ASC_DT_INT16 5

/* ---- runtime / platform --------------------------------------------------
 * Replaces rt_wrapper.cpp's device queries (GetDeviceInfoWrapper,
 * rt_wrapper.cpp:48-60) used by Launcher.get_core_num
 * (python/asc/runtime/launcher.py:110-113). */
const char* asc_last_error(void);
const char* asc_version(void);
/* Fills CU count, LDS bytes per workgroup, wavefront size and the gcnArchName
 * (arch must hold >= 64 bytes) for `device`. */
int32_t asc_device_info(int32_t device, int32_t* cu_count, int32_t* lds_bytes,
                        int32_t* wave_size, char* arch);
/* Blocks until all work on `stream` is done (rt.synchronize(),
 * python/asc/runtime/launcher.py:187). */
int32_t asc_stream_synchronize(asc_stream_t stream);

/* ---- code objects --------------------------------------------------------
 * The reference registers the binary its compiler produced and launches the
 * registered function with a packed argument blob
 * (python/asc/runtime/launcher.py:156-195, 226-238).  Here the binaries are
 * gfx950 code objects built ahead of time (pyasc_amd/lib/co/<name>.hsaco) and
 * cached per specialisation by the asc2 launch path.
 * asc_module_load       replaces DevBinaryRegisterWrapper
 *                       (python/asc/lib/runtime/rt_wrapper.cpp:115-118):
 *                       hipModuleLoad of the code object at `path` on the
 *                       current device.
 * asc_module_unload     replaces DevBinaryUnRegisterWrapper (rt_wrapper.cpp:127).
 * asc_module_get_function replaces FunctionRegisterWrapper (rt_wrapper.cpp:140-144):
 *                       the kernel named `name` (its C symbol).
 * asc_module_launch     replaces KernelLaunchWrapper (rt_wrapper.cpp:189-193):
 *                       `grid` workgroups of `block` threads on `stream`, the
 *                       kernel's arguments as one blob of `args_size` bytes laid
 *                       out as the kernel declares them (natural alignment,
 *                       8-byte pointers).  block <= 1024 and grid * block
 *                       < 2^32 (else ASC_ERR_INVALID_ARG / ASC_ERR_UNSUPPORTED). */
int32_t asc_module_load(const char* path, void** module);
int32_t asc_module_unload(void* module);
int32_t asc_module_get_function(void* module, const char* name, void** function);
int32_t asc_module_launch(void* function, uint32_t grid, uint32_t block,
                          const void* args, uint64_t args_size,
                          asc_stream_t stream);

/* A launch of one kernel of a prebuilt code object whose argument is a single
 * struct: the kernel's symbol, its grid and block, and the struct's bytes as the
 * argument blob asc_module_launch takes.  asc_flash_attention_plan,
 * asc_matmul_plan and asc_matmul_i8_plan fill it with exactly the launch their
 * library entry points make.  No counterpart in the reference, whose compiler
 * fixes the launch inside the kernel binary. */
typedef struct asc_launch_plan {
  char kernel[64];   /* NUL-terminated symbol; empty when there is nothing to launch */
  uint32_t grid;     /* workgroups (0: nothing to launch) */
  uint32_t block;    /* threads per workgroup */
  uint64_t args_size;
  uint64_t args[16]; /* the first args_size bytes are the argument blob */
} asc_launch_plan_t;

/* ---- vadd ----------------------------------------------------------------
 * asc2 vadd_kernel(x_ptr, y_ptr, out_ptr, size: int, tile_size: ConstExpr[int],
 *                  tile_per_block: ConstExpr[int])
 *   python/test/asc2/kernels/test_vadd.py:16-28 (README.md:29-40).
 * Logical block b adds tiles [(b*tpb+i)*tile, +tile) for i < tpb; the store
 * clips at `size` (lib/Conversion/LowerToAsc/LowerAscTileDataTransfer.cpp:
 * 225-271), so out[j] = x[j] + y[j] for j < min(size, grid*tpb*tile) and the
 * rest of `out` is left untouched.  dtype: ASC_DT_FLOAT32 / FLOAT16 / BFLOAT16
 * (IEEE add, RNE) or ASC_DT_INT32 (two's-complement wraparound,
 * python/test/asc2/operations/test_binary_ops.py:12,86-87). */
int32_t asc_vadd(int32_t dtype, const void* x, const void* y, void* out,
                 int64_t size, int32_t tile_size, int32_t tile_per_block,
                 int32_t grid, asc_stream_t stream);

/* ---- plain copy (bandwidth reference) --------------------------------------
 * dst[0, n_bytes) = src[0, n_bytes) with the streaming shape of the vadd kernel
 * (non-temporal 16-byte vectors, four per thread in flight).  It has no
 * counterpart among the reference's asc2 kernels: it is the copy that bounds
 * every HBM-streaming kernel here, measured beside them by the bench.  Buffers
 * and n_bytes must be multiples of 16 bytes (ASC_ERR_ALIGNMENT otherwise). */
int32_t asc_copy_bytes(const void* src, void* dst, int64_t n_bytes,
                       asc_stream_t stream);

/* ---- leaky_relu / vmuladd ------------------------------------------------------
 * asc2 leaky_relu_kernel(x_ptr, alpha: float, out_ptr, size: int,
 *                        tile_size: ConstExpr[int], tile_per_block: ConstExpr[int])
 *   python/test/asc2/kernels/test_leaky_relu.py:16-26:
 *   out = where(x >= 0, x, x * alpha); x * alpha is formed in fp32 and rounded
 *   once to the element type (RNE).
 * asc2 vmuladd_kernel(x_ptr, y_ptr, z_ptr, out_ptr, size: int,
 *                     tile_size: ConstExpr[int], tile_per_block: ConstExpr[int],
 *                     buffer_factor: ConstExpr[int])
 *   python/test/asc2/kernels/test_vmuladd.py:16-31:
 *   out = x * y + z, the product rounded to the element type before the add
 *   (no fused multiply-add).
 * Coverage as vadd: out[j] for j < min(size, grid*tpb*tile); the rest of out is
 * untouched.  dtype: ASC_DT_FLOAT32 / FLOAT16 / BFLOAT16. */
int32_t asc_leaky_relu(int32_t dtype, const void* x, float alpha, void* out,
                       int64_t size, int32_t tile_size, int32_t tile_per_block,
                       int32_t grid, asc_stream_t stream);
int32_t asc_vmuladd(int32_t dtype, const void* x, const void* y, const void* z,
                    void* out, int64_t size, int32_t tile_size,
                    int32_t tile_per_block, int32_t grid, asc_stream_t stream);

/* ---- gelu ---------------------------------------------------------------------
 * asc2 gelu_kernel(x_ptr, out_ptr, num_rows: ConstExpr, num_columns: ConstExpr,
 *                  tile_size: ConstExpr, approximate: ConstExpr)
 *   python/test/asc2/kernels/test_gelu.py:19-33.
 * fp32 [num_rows, num_cols]; each row's first tile_size columns get
 *   approximate != 0: x - x / (exp(x * (x*x*k2 + k1)) + 1),
 *                     k1 = 2*sqrt(2/pi), k2 = k1 * 0.044715
 *   approximate == 0: x * (erf(x * sqrt(0.5)) + 1) * 0.5
 * (the reference body's expressions and order).  tile_size > num_cols: the
 * reference's load pads the row with zeros and gelu is element-wise, so every
 * column of the row is computed; nothing past the row is written. */
int32_t asc_gelu_rows_f32(const float* x, float* out, int64_t num_rows,
                          int64_t num_cols, int32_t tile_size,
                          int32_t approximate, int32_t grid,
                          asc_stream_t stream);

/* ---- row softmax -----------------------------------------------------------
 * asc2 softmax_kernel(x_ptr, out_ptr, num_rows: int, num_cols: int,
 *                     tile_size: ConstExpr[int])
 *   python/test/asc2/kernels/test_softmax.py:16-27.
 * Rows i = b, b+grid, ... cover every row; each row's first `tile_size`
 * columns are replaced by exp(x - max) / sum(exp(x - max)) (the reference
 * divides, lib/Conversion/LowerToAsc/LowerArithBinary.cpp:116; here one
 * correctly rounded reciprocal per row and a multiply, within 2 ulp of the
 * quotient); columns >= tile_size are untouched.
 * tile_size > num_cols: the reference's load right-pads the tile with zeros
 * (lib/Conversion/LowerToAsc/LowerAscTileDataTransfer.cpp:181-222) and its
 * reductions count the whole tile (lib/Conversion/LowerToAsc/LowerAscTile.cpp:
 * 428-459), so row i gets exp(x - m) / s with m = max(max x, 0) and
 * s = sum exp(x - m) + (tile_size - num_cols) * exp(-m).  The reference's store
 * also spills the padded values into the next row, racing with that row's own
 * store across blocks; here each row writes its own num_cols values (the result
 * of the rows running in order on one block). */
int32_t asc_softmax_rows_f32(const float* x, float* out, int64_t num_rows,
                             int64_t num_cols, int32_t tile_size, int32_t grid,
                             asc_stream_t stream);

/* asc2 softmax_kernel(x_ptr, out_ptr, num_rows: int, num_cols: ConstExpr[int],
 *                     block_size: ConstExpr[int])
 *   python/test/asc2/kernels/test_softmax_fused.py:16-24 -> asc2.softmax
 *   (python/asc/language/tile/unary_ops.py:213-222).
 * Logical block b handles rows [b*block_size, (b+1)*block_size); rows at or
 * beyond min(num_rows, grid*block_size) are not touched. */
int32_t asc_softmax_blocks_f32(const float* x, float* out, int64_t num_rows,
                               int64_t num_cols, int32_t block_size,
                               int32_t grid, asc_stream_t stream);

/* The same two kernels on float16 x / out (asc2.softmax on an f16 tile,
 * which the op allows: python/asc/language/tile/unary_ops.py:213-222;
 * python/test/asc2/operations/test_softmax.py).  fp32 statistics (x - max in
 * fp32, libm exp, one reciprocal of the sum), each output rounded once (RNE)
 * to float16.  Same coverage rules as the float32 entries. */
int32_t asc_softmax_rows_f16(const void* x, void* out, int64_t num_rows,
                             int64_t num_cols, int32_t tile_size, int32_t grid,
                             asc_stream_t stream);
int32_t asc_softmax_blocks_f16(const void* x, void* out, int64_t num_rows,
                               int64_t num_cols, int32_t block_size,
                               int32_t grid, asc_stream_t stream);

/* The launch the four softmax entries above make, for a launcher that runs the
 * same kernels from the code object pyasc_amd/lib/co/asc2_softmax.hsaco instead
 * (the asc2 launch path does, through asc_module_launch).  No counterpart in the
 * reference, whose compiler fixes the launch inside the kernel binary.
 * dtype ASC_DT_FLOAT32 / FLOAT16; fused 0 for asc_softmax_rows_* (size is
 * tile_size), 1 for asc_softmax_blocks_* (size is block_size); the other
 * arguments and the errors are the entry's.  On success `plan` names the
 * kernel, its grid and block, and its arguments after x and out:
 *   kernel(const void* x, void* out, int64_t rows, int64_t stride,
 *          int32_t len, int32_t flag)
 * grid 0 means there is nothing to launch. */
typedef struct asc_softmax_plan {
  char kernel[32]; /* NUL-terminated symbol in asc2_softmax.hsaco */
  uint32_t grid;   /* workgroups */
  uint32_t block;  /* threads per workgroup */
  int64_t rows;
  int64_t stride;
  int32_t len;
  int32_t flag;
} asc_softmax_plan_t;
int32_t asc_softmax_plan(int32_t dtype, int32_t fused, const void* x,
                         const void* out, int64_t num_rows, int64_t num_cols,
                         int32_t size, int32_t grid, asc_softmax_plan_t* plan);

/* ---- reductions ---------------------------------------------------------------
 * asc2.reduce_sum / reduce_max / reduce_min / reduce_prod
 *   (python/asc/language/tile/reduction_ops.py:61-126) as the reference's
 *   reduction tests launch them (python/test/asc2/operations/test_reduce_ops.py:
 *   kernel, kernel_all, reduce_tile_kernel).
 * x: fp32 [rows, cols] row-major.  op: 0 sum, 1 max, 2 min, 3 prod (fp32
 * accumulation; max/min return the non-NaN operand).  dim 1: out[r] over
 * columns; dim 0: out[c] over rows; dim -1: over all elements, the result
 * written to out[0 .. out_count) (asc2.full of the scalar). */
int32_t asc_reduce_f32(int32_t op, const float* x, float* out, int64_t rows,
                       int64_t cols, int32_t dim, int64_t out_count,
                       asc_stream_t stream);

/* ---- RMS norm -------------------------------------------------------------------
 * asc2.rms_norm(input, gamma, epsilon) (python/asc/language/tile/unary_ops.py:
 * 225-237; AscendC RmsNorm) in the build's asc2-style kernel
 *   rms_norm_kernel(x_ptr, gamma_ptr, out_ptr, num_rows: int, num_cols: int,
 *                   epsilon: float, tile_size: ConstExpr[int])
 * (the reference has the op but no kernel test).  For every row, the first
 * tile_size columns get y = (x * r) * gamma[c], r = 1 / sqrt(sum(x^2) /
 * tile_size + epsilon), computed in fp32; other columns are untouched.
 * dtype ASC_DT_FLOAT32 or FLOAT16 (x and out; gamma is fp32). */
int32_t asc_rms_norm(int32_t dtype, const void* x, const float* gamma, void* out,
                     int64_t num_rows, int64_t num_cols, int32_t tile_size,
                     float epsilon, asc_stream_t stream);

/* ---- dense matmul (cube path) ------------------------------------------------
 * C[M,N] = epilogue(A[M,K] . B[K,N]) with fp32 accumulation, row-major
 * operands with leading dimensions lda/ldb/ldc (elements).
 * Covers asc2 `a @ b` / asc2.matmul (python/asc/language/tile/binary_ops.py:
 * 180-200) and zeros_acc + matmul_acc (binary_ops.py:203-221) as used by
 * python/test/asc2/kernels/test_matmul_{mnblock,tiled,fixpipe,l0c_to_l1}.py.
 * in_dtype: ASC_DT_FLOAT16 or ASC_DT_BFLOAT16 (A and B alike).
 * out_dtype: ASC_DT_FLOAT32 (plain L0C store), or ASC_DT_FLOAT16 /
 * ASC_DT_BFLOAT16 (fixpipe cast, RNE; modes F322F16/F322BF16 at
 * lib/Conversion/LowerToAsc/LowerAscTileDataTransfer.cpp:110-115).
 * relu != 0 applies max(x, 0) before the cast (fixpipe relu,
 * lib/Dialect/AscTile/Transforms/TransformStoreFixpipe.cpp:55-86). */
int32_t asc_matmul(int32_t in_dtype, int32_t out_dtype, const void* a,
                   const void* b, void* c, int64_t M, int64_t N, int64_t K,
                   int64_t lda, int64_t ldb, int64_t ldc, int32_t relu,
                   asc_stream_t stream);

/* ---- matmul with bias and activation epilogue -------------------------------
 * asc1 matmul_leakyrelu_kernel(a, b, c, bias, alpha: float, tiling, workspace)
 *   python/tutorials/05_matmul_leakyrelu/matmul_leakyrelu.py:27-70: the Matmul
 *   API with set_bias (fp32 bias[n] added to the fp32 accumulator) followed by
 *   asc.leaky_relu (python/asc/language/basic/vec_binary_scalar.py:63-66).
 * C[m,n] = cast(act(acc[m,n] + bias[n])) with acc as in asc_matmul; bias may be
 * NULL (no add); act: 0 none, 1 relu, 2 leaky relu (v >= 0 ? v : v * alpha).
 * asc_matmul(..., relu) equals asc_matmul_bias_act(..., NULL, ..., relu, 0). */
int32_t asc_matmul_bias_act(int32_t in_dtype, int32_t out_dtype, const void* a,
                            const void* b, void* c, const float* bias,
                            int64_t M, int64_t N, int64_t K, int64_t lda,
                            int64_t ldb, int64_t ldc, int32_t act, float alpha,
                            asc_stream_t stream);
/* ---- chained matmul ------------------------------------------------------------
 * asc2 matmul_kernel(a_ptr, b_ptr, c_ptr, a_shape, b_shape, c_shape, dtype)
 *   python/test/asc2/kernels/test_matmul_l0c_to_l1.py:17-30: c = a @ b in L0C,
 *   cast to dtype and moved L0C -> L1 -> L0A, then multiplied by b again.
 * t = cast(A . B) to in_dtype (RNE), C = cast(t . B) to out_dtype, both with
 * fp32 accumulation; A [M, K], B [K, N] with N == K, C [M, N], all row-major
 * and contiguous.  in_dtype: ASC_DT_FLOAT16 or ASC_DT_BFLOAT16 (A, B and the
 * intermediate alike); out_dtype as in asc_matmul.  The intermediate t
 * (M * N elements of in_dtype, row-major) is written to `workspace`, which must
 * hold workspace_bytes >= M * N * 2 bytes and must not overlap A, B or C; the
 * two matmuls run in order on `stream`, so the workspace may be reused once they
 * have run. */
int32_t asc_matmul_chained(int32_t in_dtype, int32_t out_dtype, const void* a,
                           const void* b, void* c, int64_t M, int64_t N,
                           int64_t K, void* workspace, int64_t workspace_bytes,
                           asc_stream_t stream);
/* asc_matmul_chained without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc); it has no counterpart in the reference.  The
 * intermediate lives in the library's own scratch buffer of 32 MiB per GPU (a
 * static device array, resident until the process ends), so M * N * 2 may not
 * exceed 33554432 bytes (ASC_ERR_UNSUPPORTED otherwise).  Nothing is allocated:
 * no hipMalloc, hipFree or allocating library call.  Every call on one GPU shares
 * that buffer, so the rule is: issue every call on one GPU on one stream, or order
 * the streams (an event) so that calls do not overlap; calls on one stream are
 * ordered and safe, calls that overlap (on different streams, or from several
 * threads) race on the buffer.  With ASC_NOALLOC_CHECK=1 in the environment (a
 * debugging aid; it creates one HIP event per GPU on its first checked call) a
 * call on another stream while the previous call on that GPU is still running is
 * refused with ASC_ERR_BUSY; streams under graph capture are not checked. */
int32_t asc_matmul_chained_noalloc(int32_t in_dtype, int32_t out_dtype,
                                   const void* a, const void* b, void* c,
                                   int64_t M, int64_t N, int64_t K,
                                   asc_stream_t stream);
/* The launch asc_matmul_bias_act makes with these arguments (asc_matmul(...,
 * relu) is act = relu, bias NULL), as a kernel of the code object
 * pyasc_amd/lib/co/asc2_matmul.hsaco (asc_launch_plan_t; the blob is the
 * kernel's argument struct).  Same checks and errors. */
int32_t asc_matmul_plan(int32_t in_dtype, int32_t out_dtype, const void* a,
                        const void* b, void* c, const float* bias, int64_t M,
                        int64_t N, int64_t K, int64_t lda, int64_t ldb,
                        int64_t ldc, int32_t act, float alpha,
                        asc_launch_plan_t* plan);

/* ---- int8 matmul with per-channel dequant -----------------------------------
 * asc1 matmul_kernel(a, b, c, tiling, workspace, quant_vector) with
 * Matmul.set_quant_vector
 *   (python/test/generalization/adv/test_matmul_quant.py:23-51;
 *    python/asc/language/adv/matmul.py:568-571; DEQF16 mode at
 *    lib/Conversion/LowerToAsc/LowerAscTileDataTransfer.cpp:116-117).
 * acc[m,n] = sum_k A[m,k]*B[k,n] in int32 (exact), A int8 [M,K] row-major,
 * B int8 [K,N] row-major.
 * asc_matmul_i8_i32 stores acc (int32 C, as in
 *   python/test/generalization/adv/test_matmul_iterate_all.py:106-120).
 * asc_matmul_i8_dequant_f16 stores out[m,n] = fp16_rne(fp32(acc) * s) with
 *   s = scale[n] (fp32 multiply, RNE).  trunc19 != 0 first clears the low 13
 *   mantissa bits of scale[n] (the reference golden's quant-vector handling,
 *   test_matmul_quant.py:94-106). */
int32_t asc_matmul_i8_i32(const int8_t* a, const int8_t* b, int32_t* c,
                          int64_t M, int64_t N, int64_t K, asc_stream_t stream);
int32_t asc_matmul_i8_dequant_f16(const int8_t* a, const int8_t* b,
                                  const float* scale, void* c, int64_t M,
                                  int64_t N, int64_t K, int32_t trunc19,
                                  asc_stream_t stream);
/* The launch asc_matmul_i8_i32 (dequant 0; scale and trunc19 ignored) or
 * asc_matmul_i8_dequant_f16 (dequant 1) makes, as a kernel of the code object
 * pyasc_amd/lib/co/asc2_matmul_i8.hsaco.  Same checks and errors. */
int32_t asc_matmul_i8_plan(const int8_t* a, const int8_t* b, const float* scale,
                           void* c, int64_t M, int64_t N, int64_t K,
                           int32_t dequant, int32_t trunc19,
                           asc_launch_plan_t* plan);

/* ---- flash-attention forward ---------------------------------------------------
 * No reference function exists (the reference has no attention kernel); this
 * is the asc2-style entry the build defines:
 *   flash_attention_fwd_kernel(q_ptr, k_ptr, v_ptr, o_ptr, batch, heads,
 *       seq_len, head_dim: ConstExpr[int], sm_scale: float,
 *       causal: ConstExpr[bool], block_m: ConstExpr[int], block_n: ConstExpr[int])
 * O = softmax(Q K^T * sm_scale + mask) V per (batch, head), sm_scale > 0;
 * q, k, v, o are contiguous bf16 [batch, heads, seq_len, head_dim]; fp32 online-softmax
 * statistics; causal masks keys j > query i.  lse (optional, may be NULL)
 * receives fp32 log-sum-exp per row [batch, heads, seq_len] in natural log. */
int32_t asc_flash_attention_fwd_bf16(const void* q, const void* k,
                                     const void* v, void* o, float* lse,
                                     int64_t batch, int64_t heads,
                                     int64_t seq_len, int32_t head_dim,
                                     float sm_scale, int32_t causal,
                                     asc_stream_t stream);
/* The launch asc_flash_attention_fwd_bf16 makes with these arguments, as a
 * kernel of the code object pyasc_amd/lib/co/asc2_flash_attention.hsaco.  Same
 * checks and errors (a causal plan reads the current device's CU count). */
int32_t asc_flash_attention_plan(const void* q, const void* k, const void* v,
                                 void* o, float* lse, int64_t batch,
                                 int64_t heads, int64_t seq_len,
                                 int32_t head_dim, float sm_scale,
                                 int32_t causal, asc_launch_plan_t* plan);

/* ---- element-wise tile operations ------------------------------------------------
 * The generic kernels of the reference's operation tests, one op per launch:
 *   unary   kernel(x_ptr, z_ptr, block_length, op)
 *             python/test/asc2/operations/test_unary_ops.py:35-40
 *   binary  kernel(x_ptr, y_ptr, z_ptr, block_length, fmt, op)
 *             python/test/asc2/operations/test_binary_ops.py:24-38
 *   where   where_kernel(x_ptr, y_ptr, z_ptr, op), where_scalar_kernel(x_ptr, scalar, z_ptr, op)
 *             python/test/asc2/operations/test_where.py:18-27,48-55
 * Op semantics: python/asc/language/tile/{unary_ops,binary_ops}.py; a scalar
 * operand takes the tile's dtype (utils.py:73-94).  16-bit floats compute in
 * fp32 and round once (RNE); integers wrap; integer div truncates (x / 0 = 0);
 * float max/min propagate NaN and order -0 below +0 (arith.maximumf /
 * minimumf, IEEE 754-2019).  n elements, contiguous. */
#define ASC_UNARY_ABS 0
#define ASC_UNARY_CEIL 1
#define ASC_UNARY_COS 2
#define ASC_UNARY_COSH 3
#define ASC_UNARY_ERF 4
#define ASC_UNARY_EXP 5
#define ASC_UNARY_EXP2 6
#define ASC_UNARY_FLOOR 7
#define ASC_UNARY_LOG 8
#define ASC_UNARY_LOG2 9
#define ASC_UNARY_NEGATIVE 10
#define ASC_UNARY_RELU 11
#define ASC_UNARY_RSQRT 12
#define ASC_UNARY_SIN 13
#define ASC_UNARY_SINH 14
#define ASC_UNARY_SQRT 15
#define ASC_UNARY_TAN 16
#define ASC_UNARY_TANH 17
/* out[i] = op(x[i]), fp32 (libm-accurate; rsqrt is 1 / sqrt, relu maps negative to +0). */
int32_t asc_unary_f32(int32_t op, const float* x, float* out, int64_t n,
                      asc_stream_t stream);
/* The same on float32 / float16 / bfloat16 elements: 16-bit elements widen to fp32,
 * take the fp32 op and round once (RNE).  asc2 unary ops on f16 tiles
 * (python/asc/language/tile/unary_ops.py); asc.sqrt of
 * python/test/generalization/basic/test_vsqrt.py. */
int32_t asc_unary(int32_t op, int32_t dtype, const void* x, void* out, int64_t n,
                  asc_stream_t stream);
/* dst[i] = src[i] * scalar + dst[i] (asc.axpy, python/asc/language/basic/
 * vec_ternary_scalar.py; python/test/generalization/basic/test_axpy.py):
 * float32 / float16 / bfloat16, the scalar rounded to the element type, fp32 math,
 * one rounding of the result. */
int32_t asc_axpy(int32_t dtype, const void* src, void* dst, double scalar, int64_t n,
                 asc_stream_t stream);
/* z[b, c, r] = x[b, r, c] for row-major [batch, rows, cols] of 2- or 4-byte elements
 * (asc.transpose of 16x16 tiles, python/test/generalization/basic/test_transpose.py).
 * x and z must not overlap. */
int32_t asc_transpose_batched(int32_t elem_bytes, const void* x, void* z, int64_t batch,
                              int64_t rows, int64_t cols, asc_stream_t stream);
/* dst[i] = saturate_int8(rint(src[i] * scale + offset)) (asc.adv.quant,
 * python/asc/language/adv/quantization.py:18-36; python/test/generalization/adv/
 * test_quant.py): float32 / float16 / bfloat16 src; scale and offset converted to the
 * source dtype and the multiply and add each rounded to it; ties to even; NaN -> 0. */
int32_t asc_quant_i8(int32_t dtype, const void* src, int8_t* dst, double scale, double offset,
                     int64_t n, asc_stream_t stream);

#define ASC_BIN_ADD 0
#define ASC_BIN_SUB 1
#define ASC_BIN_MUL 2
#define ASC_BIN_DIV 3
#define ASC_BIN_MAXIMUM 4
#define ASC_BIN_MINIMUM 5
#define ASC_BIN_LEFT_SHIFT 6  /* integer dtypes, scalar amount in [0, bits) */
#define ASC_BIN_RIGHT_SHIFT 7 /* arithmetic */
/* out[i] = op(a, b) with (a, b) = (x[i], y[i]) for mode 0, (x[i], s) for mode 1,
 * (s, y[i]) for mode 2; s is scalar_f for float dtypes (rounded to fp32, then to
 * the element type), scalar_i for integer dtypes (wrapped).  dtype:
 * ASC_DT_FLOAT32 / FLOAT16 / BFLOAT16 / INT32 / INT16. */
int32_t asc_binary(int32_t op, int32_t dtype, const void* x, const void* y,
                   void* out, int64_t n, int32_t mode, double scalar_f,
                   int64_t scalar_i, asc_stream_t stream);

#define ASC_CMP_EQ 0
#define ASC_CMP_NE 1
#define ASC_CMP_GT 2
#define ASC_CMP_GE 3
#define ASC_CMP_LT 4
#define ASC_CMP_LE 5
/* mode 0: out[i] = cmp(x[i], y[i]) ? x[i] : y[i];
 * mode 1: out[i] = cmp(x[i], s) ? true_value : false_value (s, true_value and
 * false_value converted to the element type as for asc_binary).  Same dtypes. */
int32_t asc_where_cmp(int32_t cmp, int32_t dtype, const void* x, const void* y,
                      void* out, int64_t n, int32_t mode, double scalar_f,
                      int64_t scalar_i, double true_value, double false_value,
                      asc_stream_t stream);

/* Tile load / op / store on a rectangle: z[r0+i, c0+j] = op(x[.], y[.]) for i < h,
 * j < w in row-major [rows, cols] tensors (1-D: rows = 1), clipped at the tensor
 * bounds as the tile store clips; op is ASC_BIN_ADD .. ASC_BIN_MINIMUM.  The
 * offsets are the tile's (asc2.load/store with offsets, or tile_id * tile shape:
 * python/asc/language/tile/memory_ops.py:24-31, 65-114); the kernels of
 * python/test/asc2/operations/test_memory_ops.py:58-92. */
int32_t asc_rect_binary(int32_t op, int32_t dtype, const void* x, const void* y,
                        void* z, int64_t rows, int64_t cols, int64_t r0,
                        int64_t c0, int64_t h, int64_t w, asc_stream_t stream);

/* z[r, c] = x[c] for r < rows, c < cols, elements of elem_bytes (1, 2, 4, 8):
 * asc2.broadcast_to from [1, cols], and with rows = 1 the data movement of
 * reshape / ravel / squeeze / expand_dims (python/asc/language/tile/shape_ops.py;
 * python/test/asc2/operations/test_shape_ops.py:47-55). */
int32_t asc_broadcast_rows(int32_t elem_bytes, const void* x, void* z,
                           int64_t rows, int64_t cols, asc_stream_t stream);

/* Atomic combine of tiles: z[j] = op(z[j], x[b * tile_len + j] + c) for b < n_tiles,
 * j < tile_len, each combine atomic (op: ASC_BIN_ADD, ASC_BIN_MAXIMUM or
 * ASC_BIN_MINIMUM; dtype float32 / float16 / bfloat16 / int32 / int16; c converted to
 * the element type as asc_binary's scalar).  Replaces the atomic store of
 * asc2.atomic_add / atomic_max / atomic_min (python/asc/language/tile/atomic_ops.py:19-33)
 * in the kernel of python/test/asc2/operations/test_atomic_ops.py:33-40, whose
 * workgroup b combines tile b.  Float add order is unspecified; the others are
 * order-independent. */
int32_t asc_atomic_tiles(int32_t op, int32_t dtype, const void* x, void* z,
                         int64_t n_tiles, int64_t tile_len, double c_f,
                         int64_t c_i, asc_stream_t stream);

/* z[i] = c for i < n, c converted to the element type as asc_binary's scalar:
 * asc2.full(...) (python/asc/language/tile/creation_ops.py:20-31) broadcast to the
 * tensor's shape and stored whole (python/test/asc2/operations/test_shape_ops.py:64-78). */
int32_t asc_fill(int32_t dtype, void* z, int64_t n, double c_f, int64_t c_i,
                 asc_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* ASC_HIP_H */
