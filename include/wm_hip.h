/*
 * wm_hip.h -- C ABI of libwm_hip, the MI355X (gfx950) device layer behind
 * whitematter's Tensor elementwise / broadcast / reduction / softmax path.
 *
 * The reference (whitematter, a CPU-only C++17 framework) has no FFI for this
 * path: its boundary is the C++ class API in core/tensor.h:12-137, whose op
 * bodies and backward closures loop over std::vector<float> on the host.
 * This header is the seam that replaces those loops.  The C++ Tensor in
 * whitematter_amd/core/tensor.{h,cpp} keeps the reference's class API and
 * calls these entry points from its op bodies and grad_fn closures; Python
 * tests and the bench call them through ctypes.  Each entry point below names
 * the reference code it replaces (file:line, relative to the reference root).
 *
 * Conventions
 *   - Every entry point returns 0 (WM_OK) or a WM_ERR_* code; wm_last_error()
 *     returns a message for the calling thread's last failure.
 *   - Tensor arguments are device pointers to contiguous row-major fp32
 *     (fp16 where named), shapes are int64 arrays of at most WM_MAX_DIMS dims.
 *     Outputs are caller-owned and must not alias inputs unless stated.
 *   - All work is enqueued on one library-owned HIP stream of the current
 *     device; calls return before the GPU finishes.  wm_d2h / wm_h2d /
 *     wm_sync synchronise with that stream.
 *   - Gradient outputs take an `accumulate` flag: 1 = "+=" (the reference's
 *     closures accumulate into zero-initialised buffers, core/tensor.cpp:911-920),
 *     0 = the buffer is known to be zero, so the kernel writes the
 *     contribution without reading the old value.  A NULL gradient pointer
 *     means "this input does not require grad".
 *   - Workspace for multi-pass reductions comes from the library's
 *     stream-ordered caching allocator (wm_alloc's pool).
 */
#ifndef WM_HIP_H
#define WM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WM_MAX_DIMS 8

enum wm_status {
    WM_OK = 0,
    WM_ERR_INVALID = 1,     /* bad argument: shape mismatch, null pointer, ... */
    WM_ERR_HIP = 2,         /* HIP runtime error */
    WM_ERR_NOMEM = 3,       /* device allocation failed */
    WM_ERR_UNSUPPORTED = 4, /* valid request this build does not implement */
    WM_ERR_IO = 5           /* a read / write callback delivered fewer bytes than asked */
};

/* Binary ops, core/tensor.cpp:897 (add), :981 (sub), :1063 (mul), :1147 (div),
 * :1385 (pow(Tensor)), :1901 (max(Tensor)), :1986 (min(Tensor)). */
enum wm_binary_op {
    WM_ADD = 0, WM_SUB = 1, WM_MUL = 2, WM_DIV = 3,
    WM_POW = 4, WM_MAX = 5, WM_MIN = 6
};

/* Unary ops.  WM_SCALE is mul(float) (core/tensor.cpp:1237-1253); div(float)
 * and neg() are WM_SCALE with p0 = 1.0f/s and p0 = -1.0f (:1255-1261). */
enum wm_unary_op {
    WM_RELU = 0,     /* :1263-1279 */
    WM_SIGMOID = 1,  /* :1281-1300 */
    WM_TANH = 2,     /* :1302-1321 */
    WM_LOG = 3,      /* :1323-1341, log(x + 1e-8f) */
    WM_EXP = 4,      /* :1343-1361 */
    WM_POWS = 5,     /* :1363-1383, pow(x, p0) */
    WM_SQRT = 6,     /* :1477-1496 */
    WM_ABS = 7,      /* :1498-1522 */
    WM_CLAMP = 8,    /* :1524-1546, clamp(x, p0, p1) */
    WM_SCALE = 9     /* :1237-1261, x * p0 */
};

/* Reductions over the middle axis of an [outer, n, inner] view. */
enum wm_reduce_op {
    WM_R_SUM = 0,     /* :1637-1707 */
    WM_R_MEAN = 1,    /* :1709-1721, sum then "/= n" in fp32 */
    WM_R_MAX = 2,     /* :1723-1810, first (lowest) index wins ties */
    WM_R_MIN = 3,     /* :1812-1899 */
    WM_R_ARGMAX = 4,  /* :2075-2145, index written as fp32 */
    WM_R_ARGMIN = 5   /* :2147-2221 */
};

/* ---- runtime ------------------------------------------------------------ */

/* Select the device and create the library stream.  Optional: every other
 * entry point initialises device 0 on first use. */
int wm_init(int device);
const char* wm_last_error(void);
/* Stream-ordered caching allocator (device memory, 256-byte aligned). */
int wm_alloc(void** ptr, size_t bytes);
int wm_free(void* ptr);
/* Return every cached block to the driver. */
int wm_empty_cache(void);
int wm_h2d(void* dst, const void* src, size_t bytes);
int wm_d2h(void* dst, const void* src, size_t bytes);
int wm_d2d(void* dst, const void* src, size_t bytes);
int wm_sync(void);
/* Number of compute units of the current device (256 on MI355X). */
int wm_device_cus(int* cus);

/* ---- measurement helpers (no reference counterpart) ---------------------- */

/* Events on the library stream bracketing enqueued work. */
int wm_timer_start(void);
int wm_timer_stop(float* elapsed_ms);
/* Per-launch event pairs: between wm_span_begin and wm_span_end, each
   kernel the library launches (up to 64) is launched with its own start and
   stop event (hipExtLaunchKernelGGL).  wm_span_end waits for the last one
   and gives the sum of the pairs' elapsed times (*kernel_ms) and, if span_ms
   is not null, the time from the first start event to the last stop event.
   The events are marker packets on either side of the dispatch, so each
   pair reads a few microseconds longer than the dispatch's own duration in a
   kernel trace.  It fails if no kernel ran.  Spans are single-threaded: a
   launch from another host thread while a span is open takes one of its
   event pairs. */
int wm_span_begin(void);
int wm_span_end(float* kernel_ms, float* span_ms, int* kernels);
/* Duration of the i-th kernel (0-based) of the last span wm_span_end closed. */
int wm_span_kernel(int i, float* ms);
/* Kernels the library has launched since the process started (every
   thread): the difference across a call is the number of dispatches it
   issued itself (copies the HIP runtime runs as kernels are not counted). */
int wm_launch_count(int64_t* count);
/* Device blocks the library's pool has handed out so far (wm_alloc and
   internal workspace); a test of an entry point that allocates nothing. */
int wm_pool_handouts(int64_t* count);
/* Plain streaming copy kernel (non-temporal loads and stores), used to
   calibrate rocprof byte counters and as the practical HBM ceiling. */
int wm_copy_kernel(float* dst, const float* src, int64_t n);
/* The same copy with ordinary cached loads and stores: calibrates the byte
   counters for kernels that read through the caches. */
int wm_copy_kernel_cached(float* dst, const float* src, int64_t n);

/* ---- fill / conversions ------------------------------------------------- */

/* out[i] = value.  Replaces the zero/one fills of Tensor's ctor and factories
 * (core/tensor.cpp:408-432) and zero_grad (:725-727). */
int wm_fill(float* out, float value, int64_t n);
/* fp32 -> fp16 with the reference's truncating conversion float_to_half
 * (core/amp.h:15-38), and fp16 -> fp32 (half_to_float, core/amp.h:40-72). */
int wm_f32_to_f16_rtz(uint16_t* out, const float* x, int64_t n);
int wm_f16_to_f32(float* out, const uint16_t* x, int64_t n);

/* ---- elementwise -------------------------------------------------------- */

/* Broadcast output shape of a and b (NumPy right-aligned rules),
 * core/tensor.cpp:338-372.  Returns WM_ERR_INVALID if not broadcastable. */
int wm_broadcast_shape(const int64_t* a_shape, int a_ndim,
                       const int64_t* b_shape, int b_ndim,
                       int64_t* out_shape, int* out_ndim);

/* out = a (op) b with broadcasting; out has the broadcast shape.
 * Replaces the fast paths (simd_add/sub/mul, :51-114) and the broadcast
 * index loops (:926-947 and the same loop in sub/mul/div/pow/max/min). */
int wm_binary(int op, float* out,
              const float* a, const int64_t* a_shape, int a_ndim,
              const float* b, const int64_t* b_shape, int b_ndim);

/* Backward of wm_binary: ga (+)= dL/da, gb (+)= dL/db, summing over the
 * broadcast dims of each operand (deterministic, fixed-order partials).
 * `out` is the forward output, read only by WM_POW's d/db = g*out*log(a);
 * when it is NULL the kernel recomputes pow(a, b) bit-identically instead of
 * reading it (one full-size read fewer).  Replaces the grad_fn closures at
 * :911-920, :956-976, :995-1005, :1039-1058, :1077-1088, :1122-1142,
 * :1163-1175, :1209-1232, :1401-1414, :1448-1472, :1917-1928, :1962-1984,
 * :2004-2015, :2049-2071. */
int wm_binary_bwd(int op, const float* g,
                  const float* a, const int64_t* a_shape, int a_ndim,
                  const float* b, const int64_t* b_shape, int b_ndim,
                  const float* out,
                  float* ga, int ga_accumulate,
                  float* gb, int gb_accumulate);

/* out = f(x) elementwise, parameters p0/p1 as listed in wm_unary_op. */
int wm_unary(int op, float* out, const float* x, int64_t n, float p0, float p1);

/* gx (+)= g * f'(x).  `x` is the forward input and `out` the forward output;
 * each op reads the one the reference closure reads (sigmoid/tanh/exp/sqrt
 * read out; relu/log/pow/abs/clamp read x).  Replaces the closures at
 * :1247-1251, :1272-1276, :1293-1298, :1314-1319, :1334-1339, :1354-1359,
 * :1374-1380, :1489-1494, :1508-1519, :1533-1544. */
int wm_unary_bwd(int op, const float* g, const float* x, const float* out,
                 float* gx, int accumulate, int64_t n, float p0, float p1);

/* ---- reductions --------------------------------------------------------- */

/* Reduce x viewed as [outer, n, inner] over n.  Outputs are [outer, inner]:
 *   val: SUM/MEAN/MAX/MIN value, or ARGMAX/ARGMIN index as fp32 (may be NULL
 *        only for MAX/MIN when idx is given);
 *   idx: for MAX/MIN/ARGMAX/ARGMIN, the winning position along n as int64
 *        (may be NULL).  Ties go to the lowest position; a NaN only wins when
 *        it is the first element, as in the reference's strict-compare scans.
 * sum(-1) / mean(-1) are outer=1, n=numel, inner=1 (core/tensor.cpp:1638);
 * dim 0 of a 2-D tensor is outer=1, n=rows, inner=cols (:1662);
 * dim 1 is outer=rows, n=cols, inner=1 (:1684); argmax/argmin over dim d of
 * an N-d tensor is outer=prod(shape[:d]), n=shape[d], inner=prod(shape[d+1:])
 * (:2096-2134). */
int wm_reduce(int op, const float* x, int64_t outer, int64_t n, int64_t inner,
              float* val, int64_t* idx);

/* wm_reduce without allocating: no counterpart in the reference; for callers
 * that cannot allocate device memory (tight serving loops, harnesses that
 * forbid hipMalloc).  It launches on the library's own stream, like every
 * entry point, so it is not meant for capture into a caller's graph.  Same
 * arguments, results
 * and errors as wm_reduce, and the same kernels; the chunk partials of a
 * split reduction live in a fixed 8 MiB device array per GPU (held until the
 * process ends) instead of the library's pool, so no device memory is taken
 * from the pool or the driver.  A reduction whose partials exceed 8 MiB
 * fails with WM_ERR_UNSUPPORTED (wm_reduce handles it).  Every call on one
 * GPU shares the array: this library orders its calls on its one stream, and
 * calls that overlap on one GPU (from another process or library instance)
 * race on it.
 * Call wm_init first: the first call on a device looks up the array's
 * address (no allocation). */
int wm_reduce_noalloc(int op, const float* x, int64_t outer, int64_t n, int64_t inner,
                      float* val, int64_t* idx);

/* Backward of wm_reduce for SUM/MEAN (gx[o,k,i] (+)= g[o,i]; the reference's
 * mean reuses sum's closure, so no 1/n, :1709-1721) and MAX/MIN
 * (gx[o,idx[o,i],i] += g[o,i]; always accumulates).  Replaces the closures
 * at :1649-1653, :1675-1681, :1697-1703, :1743-1745, :1774-1778, :1802-1806,
 * :1832-1834, :1863-1867, :1891-1895. */
int wm_reduce_bwd(int op, const float* g, const int64_t* idx,
                  int64_t outer, int64_t n, int64_t inner,
                  float* gx, int accumulate);

/* ---- softmax ------------------------------------------------------------ */

/* Row softmax / log_softmax of a [rows, cols] tensor along the last axis,
 * core/tensor.cpp:1548-1572 and :1593-1616. */
int wm_softmax_fwd(float* out, const float* x, int64_t rows, int64_t cols);
int wm_log_softmax_fwd(float* out, const float* x, int64_t rows, int64_t cols);
/* softmax: gx (+)= y * (g - sum_k g_k y_k), the closed form of the explicit
 * Jacobian loop at :1577-1588; log_softmax: gx (+)= g - exp(out) * sum_k g_k,
 * :1621-1632.  `out` is the forward output. */
int wm_softmax_bwd(const float* g, const float* out, float* gx, int accumulate,
                   int64_t rows, int64_t cols);
int wm_log_softmax_bwd(const float* g, const float* out, float* gx,
                       int accumulate, int64_t rows, int64_t cols);

/* ---- fused fp16-storage epilogue ----------------------------------------- */

/* out = tanh_(clamp((h + res) * g, lo, hi)), mean[r] = sum_c out[r,c] / cols,
 * over [rows, cols] activations h, res stored as fp16 (bits of the
 * reference's float_to_half, core/amp.h:15-38) with fp32 compute; g is a
 * per-column fp32 vector; out is written as fp16 (truncating, may be NULL)
 * and mean as fp32.  The composition of the reference ops add (:897), mul
 * with a broadcast [cols] vector (:1063), clamp (:1524), tanh_ (:1302) and
 * reshape + mean(1, keepdim) (:2250, :1709) on the half_to_float'ed inputs
 * (core/amp.h:40-72), in one pass. */
int wm_epilogue_f16_fwd(uint16_t* out, float* mean, const uint16_t* h, const uint16_t* res,
                        const float* g, int64_t rows, int64_t cols, float lo, float hi);

/* Backward of wm_epilogue_f16_fwd given dm = dL/dmean ([rows]): the chain of
 * the reference closures (mean reuses sum's closure, so no 1/cols), with the
 * forward recomputed from h, res and g.  gh, gres ([rows, cols] fp32) and
 * gg ([cols], the column sum over rows) each take an accumulate flag and may
 * be NULL. */
int wm_epilogue_f16_bwd(const float* dm, const uint16_t* h, const uint16_t* res, const float* g,
                        float* gh, int acc_h, float* gres, int acc_res, float* gg, int acc_g,
                        int64_t rows, int64_t cols, float lo, float hi);

#ifdef __cplusplus
}
#endif

#endif /* WM_HIP_H */
