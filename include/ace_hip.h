/*
 * ace_hip.h -- C-ABI of the MI355X (gfx950) mL1-ACE loss hot path.
 *
 * Two entry points replace the reference's GPU path:
 *
 *   ace_forward  replaces the forward of the reference's fastest impl,
 *                `_forward` in src/ace_kernels/impls/v6_triton.py:43-65, i.e.
 *                the fused histogram kernels `hard_hist_fused`
 *                (src/ace_kernels/kernels/hard_hist.py:186-233) /
 *                `soft_hist_fused` (kernels/soft_hist.py:229-271) followed by
 *                `epilogue_triton` (kernels/epilogue.py:93-129).
 *   ace_backward replaces `_backward` (impls/v6_triton.py:68-90), i.e.
 *                `hard_input_grad_triton` (kernels/hard_bwd.py:98-149) /
 *                `soft_input_grad_triton` (kernels/soft_bwd.py:102-163) with
 *                g = jac * grad_output fused in.
 *
 * Conventions
 *   - All pointers except `class_weight == NULL`, `stats == NULL` and the
 *     host-only arguments are device pointers on the current HIP device.
 *     With N = 0 (no voxels) `x`, `target` and `dx` may be NULL: nothing
 *     reads or writes them (the loss is then NaN, every bin being empty).
 *   - `stream` is a hipStream_t (0 = the null stream).  Every launch is
 *     asynchronous on it; no call synchronises, copies host<->device or
 *     allocates device memory, so both calls can be captured in a HIP graph.
 *   - Logits `x` are [B, C, N] contiguous (channels-first, N = prod(spatial)).
 *   - Targets are either class indices [B, N] (int64, original class
 *     numbering, ACE_TARGET_LABELS_I64) or per-channel targets [B, C, N]
 *     (float32, ACE_TARGET_ONEHOT_F32).
 *   - C' = C - 1 when include_background == 0 and C > 1, else C.
 *   - Return value: 0 on success, otherwise an ACE_E* code (see
 *     ace_error_string); a HIP launch failure returns ACE_EHIP + hipError_t.
 */
#ifndef ACE_HIP_H
#define ACE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element type of x (and of dx); ACE_F64 only through the _f64 entry points */
enum { ACE_F32 = 0, ACE_BF16 = 1, ACE_F16 = 2, ACE_F64 = 3 };
/* target layout; ACE_TARGET_ONEHOT_F64 only through the _f64 entry points */
enum { ACE_TARGET_LABELS_I64 = 0, ACE_TARGET_ONEHOT_F32 = 1, ACE_TARGET_ONEHOT_F64 = 2 };
/* binning (ACEConfig.binning) */
enum { ACE_HARD = 0, ACE_SOFT = 1 };
/* activation applied in-kernel; softmax over C == 1 must be passed as NONE */
enum { ACE_ACT_NONE = 0, ACE_ACT_SOFTMAX = 1, ACE_ACT_SIGMOID = 2 };
/* reduction over the [B, C'] per-class errors */
enum { ACE_RED_MEAN = 0, ACE_RED_SUM = 1, ACE_RED_NONE = 2 };

/* error codes */
enum {
  ACE_OK = 0,
  ACE_EINVAL = 1,       /* bad argument (null pointer, size, enum value)     */
  ACE_EUNSUPPORTED = 2, /* valid but not built: e.g. C > 64, LDS too large    */
  ACE_EWORKSPACE = 3,   /* workspace smaller than ace_workspace_bytes()       */
  ACE_ESCRATCH = 4,     /* ace_forward_noalloc: needs > ACE_NOALLOC_SCRATCH_BYTES */
  ACE_EHIP = 1000       /* + hipError_t of a failed launch                    */
};

/* ABI version of this header (incremented on any signature change). */
int ace_abi_version(void);

/* Human-readable text for a return code (static storage). */
const char* ace_error_string(int code);

/*
 * Bytes of device workspace ace_forward needs for this problem.  The
 * workspace holds ticket counters and the final fixed-point sums; its first
 * `ace_workspace_reset_bytes()` bytes (currently all of it) must be zero when
 * a call starts, and every call leaves them zero again, so repeated calls
 * reuse a workspace without clearing.  A call that needs more reset bytes than
 * earlier calls on the same buffer have left zero needs the extra bytes
 * cleared first.  Calls that share a workspace must be ordered (same stream).
 */
size_t ace_workspace_bytes(int64_t batch, int64_t channels, int64_t voxels,
                           int num_bins, int binning, int x_dtype,
                           int include_background, int target_kind);
size_t ace_workspace_reset_bytes(int64_t batch, int64_t channels,
                                 int64_t voxels, int num_bins, int binning,
                                 int x_dtype, int include_background,
                                 int target_kind);

/*
 * Forward: per-bin statistics (W, P, G) of every (b, c') slice, then the
 * epilogue (reference kernels/epilogue.py:23-82 semantics):
 *   d[b,c',k]    = P/W - G/W for non-empty bins, else 0            [B, C', K]
 *                  soft binning: `diff` holds [2, B, C', K], d rounded to
 *                  float32 (diff[0]) and d minus that rounding (diff[1]),
 *                  so that the backward's p - y - d keeps the precision of
 *                  the float64 sums; hard: [B, C', K], d in float32
 *   coef[b,c',k] = sign(d) / (K_ne * W) for non-empty bins, else 0 [B, C', K]
 *   per_class    = f * present * w_c   (f = mean |d| over non-empty bins,
 *                  NaN when every bin is empty)                    [B, C']
 *   jac          = d(sum of loss outputs) / d f                    [B, C']
 *   loss[0]      = mean / sum of per_class (unused for reduction NONE)
 * `bin_table` is the reference's float32 torch.linspace table: hard ->
 * linspace(0, 1+eps32, K+1)[1:] (K values); soft -> linspace(0, 1+eps32,
 * 2K+1)[1:] (2K values).  `centre_table` (soft only, else NULL) is
 * [-1e4, c0, c0, c1, c1, ..., c_{K-1}, c_{K-1}, 1e4] (2K+2 values).
 * `class_weight` is NULL (unweighted) or C' float32 weights.  `stats`, when not
 * NULL, receives float64 [3, B, C', K]: W, P, G.
 */
int ace_forward(const void* x, int x_dtype, const void* target,
                int target_kind, int64_t batch, int64_t channels,
                int64_t voxels, int num_bins, int binning, int activation,
                int include_background, int ignore_empty_classes,
                int reduction, int right, float empty_weight,
                const float* class_weight, const float* bin_table,
                const float* centre_table, void* workspace,
                size_t workspace_bytes, float* coef, float* diff, float* jac,
                float* per_class, float* loss, double* stats, void* stream);

/*
 * Backward: dx[b,c,n] = d loss / d x for upstream gradient `grad_output`
 * (one float32 scalar when grad_output_per_class == 0, else [B, C'] values,
 * reduction NONE).  g = jac * grad_output is formed in-kernel.  `coef`, `diff`
 * and `jac` are the forward's outputs (soft: both parts of `diff`, 2 B C' K
 * values; a caller holding only a float32 d passes zeros as its remainder);
 * `diff` may be NULL for hard binning.
 * `target` may be NULL for hard binning (the hard gradient does not use it).
 * dx has the element type of x.
 */
int ace_backward(const void* x, int x_dtype, const void* target,
                 int target_kind, int64_t batch, int64_t channels,
                 int64_t voxels, int num_bins, int binning, int activation,
                 int include_background, int right, const float* bin_table,
                 const float* centre_table, const float* coef,
                 const float* diff, const float* jac,
                 const float* grad_output, int grad_output_per_class,
                 void* dx, void* stream);

/*
 * Float64 logits: the loss and its gradient computed in double throughout,
 * outputs in double.  Replaces the reference's float64 route
 * (src/ace_kernels/impls/v6_triton.py:226-227: float64 input goes to the
 * handwritten "recompute" backward in torch, impls/v2_autograd.py:196-236,
 * with float64 softmax / sigmoid, bins and epilogue).  Arguments as
 * ace_forward / ace_backward, with x, dx, the outputs, `empty_weight`,
 * `class_weight` and `grad_output` in double; targets are int64 class ids
 * (ACE_TARGET_LABELS_I64) or a float64 [B, C, N] one-hot
 * (ACE_TARGET_ONEHOT_F64); the tables are the same float32 tables (converted
 * exactly).  The workspace is ace_workspace_bytes(..., x_dtype = ACE_F64,
 * ...), zero at the start and left zero, as for ace_forward.  Results are
 * deterministic (fixed-order float64 sums, no float atomics).  C <= 64.
 */
int ace_forward_f64(const double* x, const void* target, int target_kind,
                    int64_t batch, int64_t channels, int64_t voxels,
                    int num_bins, int binning, int activation,
                    int include_background, int ignore_empty_classes,
                    int reduction, int right, double empty_weight,
                    const double* class_weight, const float* bin_table,
                    const float* centre_table, void* workspace,
                    size_t workspace_bytes, double* coef, double* diff,
                    double* jac, double* per_class, double* loss,
                    double* stats, void* stream);
int ace_backward_f64(const double* x, const void* target, int target_kind,
                     int64_t batch, int64_t channels, int64_t voxels,
                     int num_bins, int binning, int activation,
                     int include_background, int right,
                     const float* bin_table, const float* centre_table,
                     const double* coef, const double* diff,
                     const double* jac, const double* grad_output,
                     int grad_output_per_class, double* dx, void* stream);

/*
 * Several levels of one loss in one launch per direction (deep supervision:
 * the same configuration on up to 4 resolutions of one batch).  No
 * counterpart in the reference, whose API takes one volume per call
 * (src/ace_kernels/registry.py:78-100) and which runs one call per level
 * (bench/configs/sprint11_deepsup.yaml).  Each level's outputs are
 * bit-identical to those of ace_forward / ace_backward on that level alone;
 * the launch saves the per-call latency of the small levels.  Only the
 * configurations with a fast kernel: softmax, int64 class-index targets,
 * C in {2, 3, 4, 16}, soft binning within the moments limits (else
 * ACE_EUNSUPPORTED).  The workspace holds one region per level, in order.
 */
typedef struct AceFwdLevel {
  const void* x;          /* [B, C, voxels] logits                  */
  const void* target;     /* [B, voxels] int64 class ids            */
  int64_t voxels;
  float* coef;            /* outputs as ace_forward                 */
  float* diff;
  float* jac;
  float* per_class;
  float* loss;
} AceFwdLevel;

typedef struct AceBwdLevel {
  const void* x;
  const void* target;     /* may be NULL for hard binning           */
  int64_t voxels;
  const float* coef;      /* that level's forward outputs           */
  const float* diff;
  const float* jac;
  const float* grad_output;
  void* dx;
} AceBwdLevel;

size_t ace_workspace_bytes_levels(int levels, const int64_t* voxels,
                                  int64_t batch, int64_t channels,
                                  int num_bins, int binning, int x_dtype,
                                  int include_background);
int ace_forward_levels(int levels, const AceFwdLevel* lv, int x_dtype,
                       int64_t batch, int64_t channels, int num_bins,
                       int binning, int include_background,
                       int ignore_empty_classes, int reduction, int right,
                       float empty_weight, const float* class_weight,
                       const float* bin_table, const float* centre_table,
                       void* workspace, size_t workspace_bytes, void* stream);
int ace_backward_levels(int levels, const AceBwdLevel* lv, int x_dtype,
                        int64_t batch, int64_t channels, int num_bins,
                        int binning, int include_background, int right,
                        int grad_output_per_class, const float* bin_table,
                        const float* centre_table, void* stream);

/*
 * Allocation-free forward.  No counterpart in the reference: for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The same computation and outputs
 * as ace_forward, whose kernels it launches, with the workspace taken from a
 * static device array of the library (ACE_NOALLOC_SCRATCH_BYTES, one per
 * device, held until the process ends) instead of an argument; it calls no
 * allocating routine.  The array used is the current device's (x and the
 * outputs must live there).  Before the forward it clears the bytes the
 * problem needs with a fill kernel on `stream`.  Problems whose
 * ace_workspace_bytes() exceed ACE_NOALLOC_SCRATCH_BYTES return ACE_ESCRATCH
 * before any launch.  Every call on a device shares that device's array:
 * calls that overlap on one device (different streams, or threads without an
 * order between them) race and must be serialised by the caller.
 */
#define ACE_NOALLOC_SCRATCH_BYTES ((size_t)1 << 20)
int ace_forward_noalloc(const void* x, int x_dtype, const void* target,
                        int target_kind, int64_t batch, int64_t channels,
                        int64_t voxels, int num_bins, int binning,
                        int activation, int include_background,
                        int ignore_empty_classes, int reduction, int right,
                        float empty_weight, const float* class_weight,
                        const float* bin_table, const float* centre_table,
                        float* coef, float* diff, float* jac, float* per_class,
                        float* loss, double* stats, void* stream);

/*
 * Kernel timing.  This has no counterpart in the reference, whose benchmark
 * brackets each call with events recorded on the stream
 * (src/ace_bench/timing.py:48-77); on HIP such events also time the dispatch
 * of the kernel after the work before it.  While set, every kernel that
 * ace_forward / ace_backward launch from the calling thread stamps `start`
 * (a hipEvent_t, or NULL) as it begins and `stop` as it ends
 * (hipExtLaunchKernel), so the events' elapsed time is the kernel's own
 * duration; a call that launches several kernels leaves the last one's.
 * ace_set_launch_events(NULL, NULL) turns it off.  Meant for timing eager
 * calls: turn it off before capturing calls into a HIP graph.  Returns ACE_OK.
 */
int ace_set_launch_events(void* start, void* stop);

/*
 * Measurement only; no counterpart in the reference, whose benchmark tables
 * each implementation against a bandwidth floor computed from the peak
 * (src/ace_bench/calculator.py:1-35).  These give the floor the device
 * actually reaches.
 *
 * ace_read_bytes reads every byte of a and b once (16-byte aligned, sizes
 * multiples of 16) with a plain streaming kernel and nothing else, as an
 * asynchronous launch on `stream`; `scratch` is device memory of
 * ace_read_bytes_scratch() bytes, whose contents mean nothing.  Timed like
 * the forward (ace_set_launch_events, the same cold cache), it is the read
 * rate a kernel of the forward's bytes can reach.  Returns ACE_EINVAL for
 * unaligned or null arguments, else ACE_OK or a HIP error.
 *
 * ace_set_timeline sets (or clears, with NULL) a device buffer of 8
 * uint64_t per block into which every later ace_forward launch of a fast
 * kernel (softmax with class labels) stamps the 100 MHz clock
 * (s_memrealtime) at its phases: 0 start, 1 main loop done, 2 block sums and
 * their final-sum atomics done, 3 ticket drawn, and in the blocks that run
 * an epilogue 4 epilogue done, 5 loss written, 6 soft moments' terms done,
 * 7 bins done.  The buffer must hold the launch's blocks; process-wide.
 * Returns ACE_OK.
 */
size_t ace_read_bytes_scratch(void);
int ace_read_bytes(const void* a, size_t a_bytes, const void* b, size_t b_bytes, void* scratch,
                   void* stream);
int ace_set_timeline(void* stamps);

/*
 * Test hooks.  No counterpart in the reference: they let a test force the
 * forward's cross-block failure handling from the host, with every kernel
 * still exiting normally.  Process-wide, read by each later forward call.
 * max_polls bounds the loss block's wait for another batch index's partial
 * loss word when B > 2 (default 2^20 polls; 0 gives up at once wherever the
 * word has not arrived, and that loss is then NaN; at B = 2 the two partials
 * meet in one atomic exchange and nothing waits); publish_delay makes each
 * batch epilogue sleep about 128 * publish_delay cycles (s_sleep 2 each)
 * before it publishes its word (default 0).  A negative value restores the default.  Returns
 * ACE_EINVAL for max_polls > 2^20 or publish_delay > 2^16, else ACE_OK.
 */
int ace_set_test_hooks(int max_polls, int publish_delay);

/*
 * Test hook; no counterpart in the reference.  ace_probabilities writes the
 * probabilities that every forward and backward kernel computes from x --
 * softmax over channels (max, exp, the sum in channel order, the IEEE
 * quotient), sigmoid, or x itself (ACE_ACT_*) -- as float32 [B, C, N] into
 * `p`, one asynchronous launch on `stream`.  The parity tests measure with it
 * how far the float32 rounding of the probabilities (the kernels' against
 * torch's) moves a loss or gradient.  Returns ACE_EINVAL for null pointers,
 * a bad dtype or activation, ACE_EUNSUPPORTED for C > 64, else ACE_OK or a
 * HIP error.
 */
int ace_probabilities(const void* x, int x_dtype, int64_t batch,
                      int64_t channels, int64_t voxels, int activation,
                      float* p, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ACE_HIP_H */
