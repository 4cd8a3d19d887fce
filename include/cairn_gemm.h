/*
 * cairn_gemm.h: the C ABI of libcairn_gemm_gfx950.so, the MI355X (gfx950) tensor-core GEMM library behind CAIRN's
 * mma_unordered. Plain C: pointers, sizes and one descriptor struct; no HIP or C++ types cross it. A stream is a
 * hipStream_t passed as void* (NULL: the null stream).
 *
 * Two layers:
 *
 * 1. The entries a CAIRN library would export for the multiply, with the spellings CAIRN's C header generator gives
 *    them (src/cairn/compiler/lower/header.py:215-249, 283-313): cf_NAME is the checked synchronous entry,
 *    cq_NAME(stream, ...) the same work queued on the caller's stream, NAME_device_stream binds the calling thread's
 *    synchronous device work to a caller-owned stream. They are the functions tests/soundness/test_tensor.py:31-36
 *    compiles around mma_unordered, one per storage float, for host views (cf_mma_<fmt>: the reference loop,
 *    cr::tensor::multiply, src/cairn/runtime/cairn_tensor.hpp:37-41) and device views (cf_mma_<fmt>_device,
 *    cq_mma_<fmt>_device: cr::tensor::launch, cairn_tensor.hpp:206-221). c += a * b with a m x k and b k x n
 *    row-major, c m x n row-major f32; the extents must agree with the view lengths or the process aborts.
 *
 * 2. The general entry the C++ runtime (include/cairn/cairn_tensor.hpp) calls: cairn_gemm_run with a descriptor
 *    that adds what the reference lacks: NT/TN/TT layouts, leading dimensions, bf16/f16/int32 outputs, a fused
 *    epilogue (per-row and per-column scales, bias, ReLU/GELU), int8 operands (W8A8), and the kernel choice the
 *    tile selector makes (cairn_gemm_select), which the perf model reads.
 *
 * Numerics: the reference contract (src/cairn/compiler/device/tensor.py:1-18, docs/numerics.md:53-78): every product
 * exact in f32, every output its old value plus its k products in an order the hardware picks, within
 * (k + 1) * 2^-22 * (|c| + sum |a * b|) of the exact sum. Two runs on one device give the same bits: no kernel here
 * reduces through atomics. int8 products accumulate exactly in int32. The 8-bit floats keep the contract as the
 * reference does, widened to f16 (every E4M3 and E5M2 value is one) for the f16 matrix core. The ring kernels on the
 * 8-bit float matrix core (cairn_wave_f8*, which run only where d->kernel names them) add their products in groups
 * with a narrower alignment: measured within the contract at k = 1024 on random patterns, outside it at short k
 * where one product is more than about 2^13 times the others of its group.
 */
#ifndef CAIRN_GEMM_H
#define CAIRN_GEMM_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* cairn:stated-begin */
/* Storage floats as the C header states them (header.py:276-277): the pattern and nothing else. */
typedef struct { uint16_t bits; } cairn_f16;
typedef struct { uint16_t bits; } cairn_bf16;
typedef struct { uint8_t bits; } cairn_f8e4m3;
typedef struct { uint8_t bits; } cairn_f8e5m2;

enum cairn_type {
  CAIRN_TYPE_F32 = 0,
  CAIRN_TYPE_F16 = 1,
  CAIRN_TYPE_BF16 = 2,
  CAIRN_TYPE_F8E4M3 = 3,
  CAIRN_TYPE_F8E5M2 = 4,
  CAIRN_TYPE_I8 = 5,
  CAIRN_TYPE_I32 = 6
};

enum cairn_act { CAIRN_ACT_NONE = 0, CAIRN_ACT_RELU = 1, CAIRN_ACT_GELU = 2 };

enum cairn_status {
  CAIRN_OK = 0,
  CAIRN_E_SHAPE = 1,   /* an extent is negative-free but too large, or a leading dimension too small */
  CAIRN_E_TYPE = 2,    /* an operand/output/bias type combination no kernel computes */
  CAIRN_E_KERNEL = 3,  /* the kernel id named does not exist or cannot run this problem */
  CAIRN_E_ARG = 4,     /* a null pointer where data is needed, or a bad descriptor version */
  CAIRN_E_HIP = 5,     /* the HIP runtime refused the launch */
  CAIRN_E_SCRATCH = 6  /* the split last round asked for needs more scratch than the workspace given holds */
};

#define CAIRN_GEMM_DESC_VERSION 2u /* version 1: the descriptor up to `kernel`, with no split */

/*
 * One GEMM: c = epilogue(a * b). a is m x k, stored row-major (trans_a = 0) or as its transpose, k x m row-major
 * (trans_a = 1); b is k x n, stored row-major (trans_b = 0) or as its transpose, n x k (trans_b = 1). So the
 * forward layer X.W is NN, dX = dY.W^T is NT (b = W read K-contiguous) and dW = X^T.dY is TN. c is m x n row-major.
 * A leading dimension of 0 means packed. The epilogue, each step an f32 rounding, in order:
 *   v = acc                            (f32; int8: the exact int32 sum converted to f32, nearest even)
 *   v = v * row_scale[i]               if row_scale
 *   v = v * col_scale[j]               if col_scale
 *   v = v + bias[j]                    if bias (f32 or bf16)
 *   v = relu(v) or gelu(v)             per act (GELU: 0.5 v (1 + erf(v / sqrt 2)))
 *   v = c_old + v                      if c_type is F32 and accumulate (the reference's c += a * b)
 * and stored as c_type: F32, BF16 or F16 (nearest even, overflow to infinity), or I32 (int8 operands with no
 * epilogue: the accumulator itself, bit-exact).
 */
typedef struct cairn_gemm_desc {
  uint32_t version; /* CAIRN_GEMM_DESC_VERSION */
  int32_t ab_type;  /* F16, BF16, F8E4M3, F8E5M2 or I8, for both operands */
  int32_t c_type;   /* F32, BF16, F16 or I32 */
  int32_t trans_a, trans_b;
  uint64_t m, n, k;
  uint64_t lda, ldb, ldc;
  const void* a;
  const void* b;
  void* c;
  int32_t accumulate;
  int32_t act;
  const void* bias;
  int32_t bias_type; /* F32 or BF16 */
  const float* row_scale;
  const float* col_scale;
  int32_t kernel; /* 0: the selector's choice; else an id cairn_gemm_kernel_info knows */
  /* The split last round (version 2). Where the output tiles are not a whole number of rounds of the machine's 256
   * CUs, the tiles of the last, partial round can be shared along k by `split_units` workgroups, each adding its
   * share into partial tiles in `workspace`; a fixup pass adds each tile's partials in k order (so the result's bits
   * do not depend on timing) and applies the epilogue. cairn_gemm_workspace says how many bytes the split needs.
   * workspace NULL, or split_units -1: no split. split_units 0: the selector's choice (where it pays, and within
   * workspace_bytes). split_units n > 0: about n units, n / 8 on each XCD (at least one) where the tiles divide
   * into 8 equal blocks, else n; CAIRN_E_SCRATCH where they need more than workspace_bytes, CAIRN_E_ARG where a unit
   * would reach into a third tile. The workspace is the caller's device memory, 256-byte aligned, not shared with
   * a call that may run at the same time. */
  void* workspace;
  uint64_t workspace_bytes;
  int32_t split_units;
} cairn_gemm_desc;

/* A kernel of the library: its id, what it computes and the tile it runs. */
typedef struct cairn_gemm_kernel {
  int32_t id;
  int32_t ab_type;       /* operand type it computes (F16 covers the widened 8-bit floats) */
  int32_t trans_a, trans_b;
  int32_t tile_m, tile_n, tile_k; /* output tile and k-step, in elements */
  int32_t threads;       /* per workgroup */
  int32_t lds_bytes;     /* per workgroup */
  int32_t family;        /* 0: MFMA tiled, 1: generic (any shape), 2: skinny (m <= 16, bandwidth), 4: wave
                            (256 x 256 pipelined, one wave a SIMD); 3 is not used */
  char name[48];
} cairn_gemm_kernel;

/* The selector's answer for one problem: the kernel and the work it launches. */
typedef struct cairn_gemm_choice {
  int32_t kernel;        /* id */
  int32_t family;
  int32_t tile_m, tile_n, tile_k;
  uint64_t workgroups;   /* launched */
  double waves;          /* workgroups / (CUs x workgroups resident per CU) */
  double efficiency;     /* the share of the machine the tiling keeps busy: whole-wave and edge-tile losses */
  int32_t split_tiles;   /* tiles of the split last round (0: none) */
  int32_t split_units;   /* workgroups sharing them along k */
  uint64_t split_bytes;  /* the workspace they use */
} cairn_gemm_choice;

/* Queue the GEMM on `stream`. Returns without waiting, allocates nothing and makes no stream or event, so it may be
 * captured in a HIP graph. A nonzero status means nothing was queued (CAIRN_E_HIP: the launch itself failed). */
int cairn_gemm_run(const cairn_gemm_desc* d, void* stream);

/* cairn_gemm_run for callers that cannot allocate (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc). It has no counterpart in the reference. The split last round's workspace is a scratch array the library
 * holds on each GPU (CAIRN_GEMM_STATIC_SCRATCH bytes, from the library's load to the process's end); d->workspace must
 * be NULL (else CAIRN_E_ARG). The selector's split fits the scratch; a split asked for (d->split_units > 0) that needs
 * more answers CAIRN_E_SCRATCH and queues nothing. It allocates nothing, frees nothing and makes no stream or event.
 * Every call on one GPU shares that GPU's scratch and leaves its contents to the next: two calls that may run at the
 * same time on one GPU (two streams, two threads) race on it. */
#define CAIRN_GEMM_STATIC_SCRATCH (64u << 20)
int cairn_gemm_run_static(const cairn_gemm_desc* d, void* stream);

/* The kernel cairn_gemm_run would launch for `d` (d->kernel 0) or checks that d->kernel can run it. No GPU call. */
int cairn_gemm_select(const cairn_gemm_desc* d, cairn_gemm_choice* out);

/* The workspace bytes a split last round of `d` would use with unlimited room (0 where the selector would not split
 * it, or d->split_units is -1): what a caller allocates for d->workspace. No GPU call. */
int cairn_gemm_workspace(const cairn_gemm_desc* d, uint64_t* bytes);

/* The kernel table: count, and the entry for one id (1 .. count). */
int cairn_gemm_kernel_count(void);
int cairn_gemm_kernel_info(int32_t id, cairn_gemm_kernel* out);

/* A static description of a status code. */
const char* cairn_gemm_status_string(int status);

/* The reference's whole-matrix device multiply on a stream: c += a * b, a m x k and b k x n row-major storage floats
 * of `type` (F16, BF16, F8E4M3, F8E5M2), c m x n row-major f32. What cr::tensor::launch<A> queues
 * (cairn_tensor.hpp:206-221); m, n or k of 0 queues nothing (k = 0 leaves c as it is). */
int cairn_gemm_mma(int32_t type, size_t m, size_t n, size_t k, float* c, const void* a, const void* b, void* stream);

/* The multiply's CAIRN entries (layer 1 above). cf_mma_<fmt> runs on the host, the reference loop; the device
 * variants run on the calling thread's execution context (synchronous: they return once their own stream has run
 * the work) and the cq_ variants queue on the caller's stream without waiting. cf_mma_f32 is the f32 instance of
 * the host template (config C1); the reference's checker refuses f32 operands (E-MMA) but its template computes it. */
void cf_mma_f32(size_t m, size_t n, size_t k, size_t cn, float* c, size_t an, const float* a, size_t bn,
                const float* b);
void cf_mma_f16(size_t m, size_t n, size_t k, size_t cn, float* c, size_t an, const cairn_f16* a, size_t bn,
                const cairn_f16* b);
void cf_mma_bf16(size_t m, size_t n, size_t k, size_t cn, float* c, size_t an, const cairn_bf16* a, size_t bn,
                 const cairn_bf16* b);
void cf_mma_f8e4m3(size_t m, size_t n, size_t k, size_t cn, float* c, size_t an, const cairn_f8e4m3* a, size_t bn,
                   const cairn_f8e4m3* b);
void cf_mma_f8e5m2(size_t m, size_t n, size_t k, size_t cn, float* c, size_t an, const cairn_f8e5m2* a, size_t bn,
                   const cairn_f8e5m2* b);
void cf_mma_f16_device(size_t m, size_t n, size_t k, size_t cn, float* c, size_t an, const cairn_f16* a, size_t bn,
                       const cairn_f16* b);
void cf_mma_bf16_device(size_t m, size_t n, size_t k, size_t cn, float* c, size_t an, const cairn_bf16* a,
                        size_t bn, const cairn_bf16* b);
void cf_mma_f8e4m3_device(size_t m, size_t n, size_t k, size_t cn, float* c, size_t an, const cairn_f8e4m3* a,
                          size_t bn, const cairn_f8e4m3* b);
void cf_mma_f8e5m2_device(size_t m, size_t n, size_t k, size_t cn, float* c, size_t an, const cairn_f8e5m2* a,
                          size_t bn, const cairn_f8e5m2* b);
void cq_mma_f16_device(void* stream, size_t m, size_t n, size_t k, size_t cn, float* c, size_t an,
                       const cairn_f16* a, size_t bn, const cairn_f16* b);
void cq_mma_bf16_device(void* stream, size_t m, size_t n, size_t k, size_t cn, float* c, size_t an,
                        const cairn_bf16* a, size_t bn, const cairn_bf16* b);
void cq_mma_f8e4m3_device(void* stream, size_t m, size_t n, size_t k, size_t cn, float* c, size_t an,
                          const cairn_f8e4m3* a, size_t bn, const cairn_f8e4m3* b);
void cq_mma_f8e5m2_device(void* stream, size_t m, size_t n, size_t k, size_t cn, float* c, size_t an,
                          const cairn_f8e5m2* a, size_t bn, const cairn_f8e5m2* b);

/* The calling thread's synchronous device work runs on `stream`, a hipStream_t the caller owns and keeps alive, after
 * what the caller queued there; NULL gives the thread its own stream back (header.py:296-304, cairn_exec.hpp:38-41). */
void cairn_gemm_device_stream(void* stream);

/*
 * Device quantize: q[i][j] = quantize[T](x[i][j], scale of row i) for an m x k row-major matrix x, the reference's
 * element function (src/cairn/runtime/cairn_float.hpp:116-146: x / scale in double, rounded once to nearest even,
 * saturated at T's finite range) on every element. It makes the operands of the W8A8 and fp8 GEMMs on the device:
 * activations by rows, and a weight by its output channels when stored n x k (the NT layout). The reference has no
 * such kernel; its quantize runs an element at a time in user code.
 *
 * The scale of each row, per `mode`:
 *   CAIRN_SCALE_ROW_ABSMAX  computed and written to scale[i]: the largest |x[i][j]| of the row (NaN elements left
 *                           out) divided by T's largest finite value (127, 448 for E4M3, 57344 for E5M2) in f32,
 *                           nearest even; 1 for a row of zeros. The row is read once (longer rows than 8192
 *                           elements: once from HBM, once from cache).
 *   CAIRN_SCALE_ROW         read from scale[i];
 *   CAIRN_SCALE_TENSOR      scale[0] for every row.
 * Where the reference traps, a kernel cannot: a row whose scale is not positive and finite (a given one, or one
 * computed from a row holding an infinity) is written as zeros and CAIRN_QUANT_BAD_SCALE is ORed into *status; a NaN
 * quantized to int8 is written as 0 and CAIRN_QUANT_NAN is ORed in. status may be NULL. Queued on `stream` like
 * cairn_gemm_run: no allocation, no stream or event, no wait.
 */
enum cairn_scale_mode { CAIRN_SCALE_ROW_ABSMAX = 0, CAIRN_SCALE_ROW = 1, CAIRN_SCALE_TENSOR = 2 };
enum cairn_quant_status { CAIRN_QUANT_BAD_SCALE = 1, CAIRN_QUANT_NAN = 2 };

#define CAIRN_QUANTIZE_DESC_VERSION 1u

typedef struct cairn_quantize_desc {
  uint32_t version; /* CAIRN_QUANTIZE_DESC_VERSION */
  int32_t x_type;   /* F32, F16 or BF16 */
  int32_t q_type;   /* I8, F8E4M3 or F8E5M2 */
  int32_t mode;     /* cairn_scale_mode */
  uint64_t m, k;     /* m < 2^31, k <= 2^28 */
  uint64_t ldx, ldq; /* elements; 0: packed */
  const void* x;
  void* q;
  float* scale;      /* m floats (ROW_ABSMAX: written; ROW: read), or 1 (TENSOR) */
  int32_t* status;   /* device word or NULL */
} cairn_quantize_desc;

int cairn_quantize_run(const cairn_quantize_desc* d, void* stream);

/* The kernel cairn_quantize_run launches for `d`, by name (as a profiler lists it, with its types and rows a
 * workgroup, e.g. "quantize_fast<bf16, i8, 4>"), or NULL where it refuses `d` or has nothing to launch. No GPU call. */
const char* cairn_quantize_kernel(const cairn_quantize_desc* d);
/* cairn:stated-end */

/*
 * The interface identity, derived as CAIRN's header generator derives a library's (header.py:280-285):
 * cairn_interface_<library>_<the first 16 hex digits of the SHA-256 of the stated interface>, the text between the
 * two cairn:stated markers above, byte for byte. The library built with this header defines the symbol, and the
 * header refers to it, so a program built against another version of this header fails to link instead of passing
 * descriptors whose fields have moved. cairn_amd/identity.py recomputes it (and rewrites this line with --write);
 * the build refuses a header whose identity is stale. A translation unit that uses the header's types without the
 * library (a host-only test machine, or an emulated build: CAIRN_EMULATE) defines CAIRN_GEMM_UNLINKED.
 */
#define CAIRN_GEMM_IDENTITY cairn_interface_gemm_gfx950_15b0d41353760eb5
extern const char CAIRN_GEMM_IDENTITY[];
#if !defined(CAIRN_GEMM_UNLINKED) && !defined(CAIRN_EMULATE)
static const char* const cairn_interface_of_gemm_gfx950 __attribute__((used)) = CAIRN_GEMM_IDENTITY;
#endif

#ifdef __cplusplus
}
#endif
#endif /* CAIRN_GEMM_H */
