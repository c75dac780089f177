/*
 * tl_hip.h -- C ABI of tl_hip, the MI355X (gfx950) backend for TL's quantized
 * LLM-inference hot path.
 *
 * Conventions (the reference's FFI conventions, crates/tl_runtime/src/device_ffi.rs):
 *   - Tensor-returning calls return a NEW handle (reference count 1) owned by the caller;
 *     input handles are borrowed (ffi_helpers.rs:43-66).  Release with tl_hip_tensor_release.
 *   - On failure a call returns NULL (or a non-zero status) and records a thread-local
 *     message readable with tl_hip_last_error() -- the LAST_ERROR + sentinel convention of
 *     device_ffi.rs:22-80, 106-113.  Nothing aborts or panics.
 *   - Status codes mirror tl_backend::BackendError (crates/tl_backend/src/error.rs:7-17).
 *   - All device work is ordered on one HIP stream per process (tl_hip_stream) unless the
 *     calling thread redirects it (tl_hip_set_stream) or a launcher is given a stream; calls
 *     that return data to the host synchronise the stream they ran on.
 *   - Device memory is cached and reused in stream order: releasing a tensor (or any freed
 *     temporary) "frees it on" the calling thread's current stream, and that memory is reused
 *     at once by later work on the same stream, by work on other streams only after the
 *     work queued before the release has completed.  Release a tensor on the stream of its
 *     last use, or synchronise that stream first.
 * Every entry point names the reference interface it replaces.
 */
#ifndef TL_HIP_H
#define TL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TL_HIP_MAX_RANK 8

/* status codes: 0 = ok, else BackendError variant (error.rs:7-17) */
#define TL_HIP_OK 0
#define TL_HIP_ERR_SHAPE 1     /* ShapeMismatch */
#define TL_HIP_ERR_DEVICE 2    /* DeviceError */
#define TL_HIP_ERR_ALLOC 3     /* AllocationError */
#define TL_HIP_ERR_NULL 4      /* NullPointerError */
#define TL_HIP_ERR_INTERNAL 5  /* InternalError */
#define TL_HIP_ERR_INDEX 6     /* IndexOutOfBounds */
#define TL_HIP_ERR_TYPE 7      /* TypeMismatch */
#define TL_HIP_ERR_ARG 8       /* ArgumentError */

/* element types of device tensors (tl_backend DType subset, dtype.rs:5-30) */
#define TL_HIP_F32 0
#define TL_HIP_F16 1

/* GGML type ids accepted for quantized weights (quantized.rs:10-22; gguf.rs:157-168) */
#define TL_HIP_GGML_F32 0
#define TL_HIP_GGML_F16 1
#define TL_HIP_GGML_Q4_0 2
#define TL_HIP_GGML_Q8_0 8
#define TL_HIP_GGML_Q4_K 12
#define TL_HIP_GGML_Q6_K 14

typedef struct tl_hip_tensor tl_hip_tensor;   /* GpuTensor (tl_backend tensor.rs:7-55) */
typedef struct tl_hip_qtensor tl_hip_qtensor; /* QTensor + gpu_raw_cache (quantized.rs:29-40) */
typedef struct tl_hip_llama tl_hip_llama;     /* decoder state of chatbot.tl (see below) */

/* ---------------------------------------------------------------- runtime -------- */
/* Last error of the calling thread (device_ffi.rs:22-80 LAST_ERROR); "" when none. */
const char* tl_hip_last_error(void);
int tl_hip_last_status(void);
void tl_hip_clear_error(void);
/* Selects the device and creates the library stream.  Optional: every other call
 * initialises device 0 on first use (the reference's global device, tl_cuda device.rs:19-86). */
int tl_hip_init(int device);
int tl_hip_device_count(void);
/* Library stream as a hipStream_t (GpuStream, tl_backend stream.rs:12-31). */
void* tl_hip_stream(void);
/* Redirects the calling thread's library work to a caller stream (NULL restores the library
 * stream).  Stream priorities other than the default are not supported. */
int tl_hip_set_stream(void* hip_stream);
int tl_hip_synchronize(void);
/* Device-memory plumbing for C callers and tests. */
void* tl_hip_malloc(size_t bytes);
int tl_hip_free(void* p);
int tl_hip_memcpy_h2d(void* dst, const void* src, size_t bytes);
int tl_hip_memcpy_d2h(void* dst, const void* src, size_t bytes);
int tl_hip_memcpy_d2d(void* dst, const void* src, size_t bytes);
/* hipEvent timing on the library stream. */
void* tl_hip_event_create(void);
int tl_hip_event_record(void* ev);
int tl_hip_event_elapsed_ms(void* start, void* stop, float* ms);
int tl_hip_event_destroy(void* ev);
/* Enqueues a one-wavefront kernel that idles for `us` microseconds (at most 100000) on the
 * library stream, so that work enqueued behind it is timed back-to-back on the GPU rather
 * than at the host's launch rate.  Timing plumbing; no reference counterpart. */
int tl_hip_stall(uint32_t us);
/* Fault injection for error-path tests: the allocation after `after` more successful ones
 * fails with AllocationError (after < 0 disables).  No reference counterpart; the reference
 * panics on allocation failure (tl_cuda tensor.rs:128-141). */
int tl_hip_debug_fail_alloc(int64_t after);

/* ---------------------------------------------------------------- tensors -------- */
/* IDevice::tensor_new (crates/tl_backend/src/device.rs:21-26): f32 host data -> device. */
tl_hip_tensor* tl_hip_tensor_new(const float* host, const int64_t* shape, int rank);
/* tensor_new for f16 payloads given as raw IEEE binary16 bits (KV-cache / f16 inputs). */
tl_hip_tensor* tl_hip_tensor_new_f16(const uint16_t* host, const int64_t* shape, int rank);
/* IDevice::tensor_zeros (device.rs:34-39). */
tl_hip_tensor* tl_hip_tensor_zeros(const int64_t* shape, int rank, int dtype);
/* IDevice::tensor_release / tensor_acquire (device.rs:213-214; ffi_helpers.rs:49-66). */
int tl_hip_tensor_release(tl_hip_tensor* t);
tl_hip_tensor* tl_hip_tensor_acquire(tl_hip_tensor* t);
/* IDevice::tensor_to_vec_f32 (device.rs:83): copies numel f32 values (f16 is widened). */
int tl_hip_tensor_to_host(const tl_hip_tensor* t, float* out, int64_t numel);
int tl_hip_tensor_rank(const tl_hip_tensor* t);
int tl_hip_tensor_shape(const tl_hip_tensor* t, int64_t* shape_out);
int64_t tl_hip_tensor_numel(const tl_hip_tensor* t);
int tl_hip_tensor_dtype(const tl_hip_tensor* t);
/* IDevice::tensor_data (device.rs:224): the device pointer. */
void* tl_hip_tensor_data(const tl_hip_tensor* t);
/* IDevice::tensor_reshape_new (device.rs:367-371): a new handle with the new shape
 * (data copied on device). */
tl_hip_tensor* tl_hip_tensor_reshape(const tl_hip_tensor* t, const int64_t* shape, int rank);

/* ------------------------------------------------------- quantized weights -------- */
/* Upload of one GGUF tensor: gguf.rs:129-189 hands over the raw block bytes with the
 * row-major shape [n, k]; QTensor::dequantize_to_tensor's size checks apply
 * (quantized.rs:182-260 for Q4_0 / Q8_0, 268-400 for Q6_K / Q4_K; rows must hold whole
 * blocks: k % 32, k % 256 for the K-quants).  The blocks are repacked once into the device
 * residency format (the gpu_raw_cache of system.rs:316-331, which the reference keeps for
 * Q4_K / Q6_K); F16/F32 are rejected (TypeMismatch). */
tl_hip_qtensor* tl_hip_qtensor_new(int ggml_type, const uint8_t* data, size_t nbytes,
                                   const int64_t* shape, int rank);
int tl_hip_qtensor_release(tl_hip_qtensor* q);
/* QTensor::dequantize_to_tensor (quantized.rs:117-165): f32 [n, k] on the device. */
tl_hip_tensor* tl_hip_qtensor_dequantize(const tl_hip_qtensor* q);
/* tl_qtensor_matmul (crates/tl_runtime/src/system.rs:180-382): y = x . W^T with x
 * [..., k] f32 and W [n, k] quantized; y is [..., n].  Fused dequant + product for all four
 * types (the reference fuses Q4_K / Q6_K on its GPU backends, cuda_mul_mv_q4_k /
 * cuda_mul_mv_q6_k at device_ffi.rs:1803-1833); m <= 4 rows take the matvec kernel, larger
 * m the tiled GEMM. */
tl_hip_tensor* tl_hip_qtensor_matmul(const tl_hip_tensor* x, const tl_hip_qtensor* q);
/* Same with the f16-MFMA prefill GEMM for m > 4 (dequant -> f16 LDS tiles -> MFMA,
 * f32 accumulate); tolerance class "f16 path".  Q4_0, Q8_0 and Q4_K are dequantized in
 * registers; a Q4_K tensor's first call builds its per-32-weight (d sc, -dmin m) f16 pairs
 * (4 bytes per 32 weights, kept until the tensor is released).  Q6_K weights are first
 * dequantized into an f16 workspace in the MFMA operand order. */
tl_hip_tensor* tl_hip_qtensor_matmul_f16(const tl_hip_tensor* x, const tl_hip_qtensor* q);

/* ---------------------------------------------------------------- GGUF files ----- */
/* The tensor map of a GGUF file (OpaqueTensorMap of tensor_map.rs, filled by tl_gguf_load). */
typedef struct tl_hip_gguf tl_hip_gguf;
/* tl_gguf_load (crates/tl_runtime/src/gguf.rs:34-196): maps the file and reads the GGUF v2 / v3
 * header ("GGUF" or byte-swapped "FUGG"), metadata and tensor table; data start = end of the
 * tensor table rounded up to general.alignment (default 32).  Shapes as gguf.rs:129-136
 * (trailing 1s trimmed, reversed to row-major); tensors of types outside F32, F16, Q4_0,
 * Q4_1, Q5_0, Q5_1, Q8_0, Q8_1, Q4_K, Q6_K or with data past the end of the file are skipped
 * (gguf.rs:157-182).  NULL + ArgumentError when the file cannot be opened or decoded. */
tl_hip_gguf* tl_hip_gguf_open(const char* path);
/* tl_tensor_map_free (tensor_map.rs:68-77): also drops the map's references to the weight
 * residencies handed out by tl_hip_gguf_get_quantized. */
int tl_hip_gguf_close(tl_hip_gguf* g);
int64_t tl_hip_gguf_tensor_count(const tl_hip_gguf* g);
const char* tl_hip_gguf_tensor_name(const tl_hip_gguf* g, int64_t i);
/* ggml type, row-major shape (up to TL_HIP_MAX_RANK entries), rank and data bytes of a tensor. */
int tl_hip_gguf_tensor_info(const tl_hip_gguf* g, const char* name, int* ggml_type, int64_t* shape,
                            int* rank, uint64_t* nbytes);
/* The tensor's bytes inside the mapped file (valid until tl_hip_gguf_close). */
const uint8_t* tl_hip_gguf_tensor_data(const tl_hip_gguf* g, const char* name, uint64_t* nbytes);
/* Metadata (GGUF key/value section): numeric values as double, strings as text. */
int tl_hip_gguf_meta_f64(const tl_hip_gguf* g, const char* key, double* out);
const char* tl_hip_gguf_meta_str(const tl_hip_gguf* g, const char* key);
/* tl_tensor_map_get_quantized (tensor_map.rs:279-301): the quantized weight handle; its
 * device residency is built from the mapped bytes on the first request and shared by later
 * ones (each call returns one more reference, released with tl_hip_qtensor_release). */
tl_hip_qtensor* tl_hip_gguf_get_quantized(tl_hip_gguf* g, const char* name);
/* tl_tensor_map_get (tensor_map.rs:110-150): an f32 device tensor -- F32 data as stored, F16
 * converted (quantized.rs:167-180), quantized types dequantized (quantized.rs:117-165). */
tl_hip_tensor* tl_hip_gguf_get(tl_hip_gguf* g, const char* name);

/* ---------------------------------------------------------------- raw launchers --- */
/* Kernel ABI in the style of launch_mul_mv_q4_k_kernel (crates/tl_cuda/src/cuda_kernels/
 * autograd.cu:2904-2924): device pointers + dims + stream, returns a status.  `w` is a
 * quantized weight handle (its residency buffers); x is [m, k] f32, y is [m, n] f32.
 * stream NULL = library stream. */
int tl_hip_launch_quant_matvec(const tl_hip_qtensor* w, const float* x, float* y, int64_t m,
                               void* stream);
int tl_hip_launch_quant_gemm(const tl_hip_qtensor* w, const float* x, float* y, int64_t m,
                             int use_f16_mfma, void* stream);
/* The one-launch floor of the decode matvec over w: the loads of the m = 1 matvec -- its
 * launch plan and access pattern, quant bytes and scale data -- with no arithmetic, reduction
 * or store; the time a matvec of w cannot beat.  Timing plumbing for the roofline; no
 * reference counterpart. */
int tl_hip_read_floor(const tl_hip_qtensor* w, void* stream);
/* Allocation-free variant of tl_hip_launch_quant_gemm (no counterpart in the reference): for
 * callers that cannot allocate device memory -- code under hipGraph capture, serving loops
 * that forbid hipMalloc.  Same arguments and results; calls no hipMalloc / hipFree.  The f16
 * MFMA path keeps its workspace (X converted to f16: m * k * 2 bytes rounded up to 256, then
 * the split-K partial tiles of 17-64-row inputs; inputs of up to 16 rows need none) in a
 * fixed 32 MiB device array per GPU, held until
 * the process ends; calls needing more are ArgumentError, as are weights that need an f16 copy
 * for the MFMA path (Q6_K, and Q4_K before its first f16 GEMM through an allocating entry).
 * The f32 path (use_f16_mfma = 0) needs no workspace.  Every call on a GPU shares that array:
 * calls on one stream are ordered, calls that overlap on different streams race.  Under
 * hipGraph capture: the array's address is looked up at library initialisation, and the
 * first library call on a caller stream (which synchronises the library stream once) must
 * precede the capture -- captured first, it is ArgumentError. */
int tl_hip_launch_quant_gemm_noalloc(const tl_hip_qtensor* w, const float* x, float* y, int64_t m,
                                     int use_f16_mfma, void* stream);
/* Tile plan of the calling thread's last f16-MFMA GEMM launch: rows and columns of one
 * workgroup's output tile and the number of K splits (1 = unsplit).  Instrumentation for the
 * parity tests (which kernel variant ran); no reference counterpart. */
int tl_hip_debug_last_gemm_plan(int* tile_m, int* tile_n, int* k_splits);

/* ------------------------------------------------------------ tensor operators --- */
/* IDevice::tensor_matmul (device.rs:258; tl_cpu tensor.rs:1248-1313): [.., m, k] x
 * [.., k, n] (b batched only when its rank > 2) or 1-D operands. */
tl_hip_tensor* tl_hip_tensor_matmul(const tl_hip_tensor* a, const tl_hip_tensor* b);
/* IDevice::tensor_transpose_2d (device.rs:513; tensor.rs:902-941) */
tl_hip_tensor* tl_hip_tensor_transpose_2d(const tl_hip_tensor* a);
/* IDevice::tensor_transpose (device.rs:378-383; tensor.rs:902-941) */
tl_hip_tensor* tl_hip_tensor_transpose(const tl_hip_tensor* a, int64_t dim0, int64_t dim1);
/* IDevice::tensor_rms_norm (device.rs:428-433; tl_cpu ffi.rs:2444-2486):
 * (x / sqrt(mean(x^2) + eps)) * w over the last dim; w may be NULL. */
tl_hip_tensor* tl_hip_tensor_rms_norm(const tl_hip_tensor* x, const tl_hip_tensor* w, float eps);
/* IDevice::tensor_rope_new_cos / _sin (device.rs:434-445; ffi.rs:2589-2629): table
 * [seq_len, dim] with each pair's value duplicated. */
tl_hip_tensor* tl_hip_tensor_rope_new_cos(int64_t dim, int64_t seq_len, float base);
tl_hip_tensor* tl_hip_tensor_rope_new_sin(int64_t dim, int64_t seq_len, float base);
/* IDevice::tensor_apply_rope (device.rs:446-451; ffi.rs:2631-2686): interleaved pairs,
 * every vector rotated by the first row of the given tables. */
tl_hip_tensor* tl_hip_tensor_apply_rope(const tl_hip_tensor* x, const tl_hip_tensor* cos_t,
                                        const tl_hip_tensor* sin_t);
/* Position-aware variant (no reference counterpart on tl_cpu; the tl_cuda kernel's
 * per-token rows, autograd.cu:1196-1227, with tl_cpu's interleaved pairs): vector v of
 * token t = v / vectors_per_token uses table row pos0 + t. */
tl_hip_tensor* tl_hip_tensor_apply_rope_pos(const tl_hip_tensor* x, const tl_hip_tensor* cos_t,
                                            const tl_hip_tensor* sin_t, int64_t pos0,
                                            int64_t vectors_per_token);
/* IDevice::tensor_silu (device.rs:310; ffi.rs:2097-2113) */
tl_hip_tensor* tl_hip_tensor_silu(const tl_hip_tensor* x);
/* IDevice::tensor_add / tensor_mul / tensor_sub / tensor_div (device.rs:253-256;
 * tensor.rs:549-621), numpy broadcasting. */
tl_hip_tensor* tl_hip_tensor_add(const tl_hip_tensor* a, const tl_hip_tensor* b);
tl_hip_tensor* tl_hip_tensor_mul(const tl_hip_tensor* a, const tl_hip_tensor* b);
tl_hip_tensor* tl_hip_tensor_sub(const tl_hip_tensor* a, const tl_hip_tensor* b);
tl_hip_tensor* tl_hip_tensor_div(const tl_hip_tensor* a, const tl_hip_tensor* b);
/* IDevice::tensor_scale (device.rs:285; ffi.rs:2083-2094) */
tl_hip_tensor* tl_hip_tensor_scale(const tl_hip_tensor* x, float s);
/* IDevice::tensor_softmax (device.rs:317; tensor.rs:1065-1092), negative dim allowed */
tl_hip_tensor* tl_hip_tensor_softmax(const tl_hip_tensor* x, int64_t dim);
/* IDevice::tensor_new_causal_mask (device.rs:53; ffi.rs:3184-3196) */
tl_hip_tensor* tl_hip_tensor_new_causal_mask(int64_t size);
/* IDevice::tensor_narrow (device.rs:391-397; tensor.rs:989-1015) */
tl_hip_tensor* tl_hip_tensor_narrow(const tl_hip_tensor* x, int64_t dim, int64_t start,
                                    int64_t len);
/* IDevice::tensor_cat (device.rs:398; tensor.rs:1021-1063), two operands */
tl_hip_tensor* tl_hip_tensor_cat(const tl_hip_tensor* a, const tl_hip_tensor* b, int64_t dim);
/* IDevice::tensor_repeat_interleave (device.rs:409-414; tensor.rs:1178-1200) */
tl_hip_tensor* tl_hip_tensor_repeat_interleave(const tl_hip_tensor* x, int64_t repeats,
                                               int64_t dim);
/* IDevice::tensor_embedding (device.rs:418-425; tensor.rs:1094-1112): ids hold f32 token
 * ids; an id outside [0, vocab) is IndexOutOfBounds. */
tl_hip_tensor* tl_hip_tensor_embedding(const tl_hip_tensor* weight, const tl_hip_tensor* ids);
/* IDevice::tensor_sample (device.rs:349; tensor.rs:1626-1680) over all elements of logits:
 * returns [1] holding the chosen index.  temp <= 0: the argmax (last index among equal
 * maxima).  Otherwise (a NaN temp included) top-p sampling of softmax(logits / temp): the
 * indices by descending probability (equal probabilities in index order), cut after the
 * first place where the running sum exceeds top_p, and the first place whose running sum
 * reaches u * (running sum at the cut) is chosen, u a uniform draw in [0, 1) from this
 * library's per-thread generator (the reference draws from rand::thread_rng).  A NaN or
 * infinite logits / temp gives index 0, as in the reference.  Empty logits: InternalError. */
tl_hip_tensor* tl_hip_tensor_sample(const tl_hip_tensor* logits, float temp, float top_p);
/* tl_hip_tensor_sample with the uniform draw given (0 <= u < 1, else ArgumentError).  No
 * counterpart in the reference, whose draw cannot be fixed: for callers and tests that
 * replay a choice.  Running sums are exact (fixed point), so the choice equals the
 * reference's wherever r = u * cutoff and top_p are not within the reference's f32 rounding
 * of a running sum. */
tl_hip_tensor* tl_hip_tensor_sample_uniform(const tl_hip_tensor* logits, float temp, float top_p,
                                            double u);
/* Seeds the calling thread's generator of tl_hip_tensor_sample (splitmix64; a draw is its
 * top 53 bits times 2^-53).  Unseeded threads start from OS entropy.  No counterpart in the
 * reference (rand::thread_rng is not seedable): for reproducible sampling runs. */
void tl_hip_sample_seed(uint64_t seed);
/* argmax over all elements (tensor.rs:841-846), last index among equal maxima. */
int64_t tl_hip_tensor_argmax_all(const tl_hip_tensor* x);
/* IDevice::tensor_repetition_penalty (device.rs:194-199; tl_cpu device_impl.rs:967-1001) */
tl_hip_tensor* tl_hip_tensor_repetition_penalty(const tl_hip_tensor* logits,
                                                const tl_hip_tensor* tokens, double penalty);

/* GpuFusedOps (crates/tl_backend/src/fused_ops.rs:15-57; tl_cpu fused_ops.rs:15-131) */
tl_hip_tensor* tl_hip_fused_silu_mul(const tl_hip_tensor* gate, const tl_hip_tensor* up);
tl_hip_tensor* tl_hip_fused_rms_norm(const tl_hip_tensor* x, const tl_hip_tensor* w, float eps);
tl_hip_tensor* tl_hip_fused_add_rms_norm(const tl_hip_tensor* x, const tl_hip_tensor* residual,
                                         const tl_hip_tensor* w, float eps);
/* GpuFusedOps::fused_rotary_emb (fused_ops.rs:38-42; tl_cpu fused_ops.rs:87-108): half-split
 * pairs rotated by cos / sin of freqs[p] as tl_cpu computes it -- for inputs longer than one
 * head vector the reference's pair indexing (base = id - id % (head_dim / 2)) overlaps
 * consecutive vectors, and this entry returns the same values.  ArgumentError when
 * head_dim < 2, freqs has fewer than head_dim / 2 entries or x fewer than head_dim. */
tl_hip_tensor* tl_hip_fused_rotary_emb(const tl_hip_tensor* x, const tl_hip_tensor* freqs, int64_t head_dim);
/* GpuFusedOps::fused_add_relu (fused_ops.rs:47-51; tl_cpu fused_ops.rs:110-120):
 * max(a + b, 0); ShapeMismatch when the element counts differ. */
tl_hip_tensor* tl_hip_fused_add_relu(const tl_hip_tensor* a, const tl_hip_tensor* b);
/* GpuFusedOps::fused_bias_gelu (fused_ops.rs:53-56; tl_cpu fused_ops.rs:122-131 with gelu at
 * 20-22): gelu(x + bias[i % len(bias)]) with tl_cpu's constant 2/sqrt(pi). */
tl_hip_tensor* tl_hip_fused_bias_gelu(const tl_hip_tensor* x, const tl_hip_tensor* bias);

/* IDevice::tensor_scaled_dot_product_attention (crates/tl_backend/src/device.rs:180-186; tl_cpu
 * device_impl.rs:775-872): q [batch, heads, seq_q, d_k], [heads, seq_q, d_k] or [seq_q, d_k];
 * k [.., seq_k, d_k] and v [.., seq_k, d_v] with the same leading dimensions (one KV head per
 * query head); all f32.  scores = q k^T * (1 / sqrt(d_k)); mask (f32, may be NULL) is read as
 * flat [seq_q, seq_k] data shared by every (batch, head): a score whose mask element exists and
 * equals 0 becomes -1e9, any other mask value leaves it unchanged; softmax over the keys; out
 * [.., seq_q, d_v] = softmax . v.  f32 arithmetic (tolerance class "f32 path"). */
tl_hip_tensor* tl_hip_tensor_scaled_dot_product_attention(const tl_hip_tensor* q, const tl_hip_tensor* k,
                                                          const tl_hip_tensor* v, const tl_hip_tensor* mask);

/* Single-query decode attention over an f16 KV cache: the chatbot's
 * transpose/cat_4d/repeat_interleave/matmul_4d/scale/softmax/matmul_4d chain
 * (examples/apps/tinyllama/chatbot.tl:63-87) for sl = 1, in one fused split-L kernel pair.
 *   q [B, Hq, D] f32;  k, v [B, Hkv, Lmax, D] f16 with the first L rows valid;
 *   out [B, Hq, D] f32;  query head h reads KV head h / (Hq / Hkv). */
tl_hip_tensor* tl_hip_attention_decode(const tl_hip_tensor* q, const tl_hip_tensor* k,
                                       const tl_hip_tensor* v, int64_t L, float scale);
/* Whether split kernels may merge their partial results inside the same launch, the
 * workgroup that finishes a unit last merging it (default 1): decode attention's split records
 * per (batch item, KV head), the short-input GEMMs' K-split slices per tile.  on = 0 selects
 * the second merge kernel, 1 the one-launch form; both return the previous setting.  on < 0
 * changes nothing and returns whether one-launch merges are in effect now (the setting is 1
 * and no stream but the library's has run library work).  Instrumentation for the parity
 * tests, which run both forms; no reference counterpart. */
int tl_hip_debug_one_launch_merge(int on);
/* Causal prefill attention over an f16 KV cache: the same chatbot chain for sl > 1 with the
 * causal mask (Tensor::new_causal_mask + add_4d, chatbot.tl:76-87), in one f16-MFMA kernel.
 *   q [n, Hq, D] f32 holds the queries of positions pos0 .. pos0 + n - 1;
 *   k, v [Hkv, Lmax, D] f16 with rows 0 .. pos0 + n - 1 valid; out [n, Hq, D] f32;
 *   query i attends rows 0 .. pos0 + i; query head h reads KV head h / (Hq / Hkv).
 * Covers D in {64, 128} with Hq / Hkv in {4, 8} (ArgumentError otherwise); the chatbot
 * itself only prefills at pos0 = 0, later positions serve chunked prompts.  q, P, K and V
 * enter the MFMAs in f16; scores, softmax and sums in f32. */
tl_hip_tensor* tl_hip_attention_prefill(const tl_hip_tensor* q, const tl_hip_tensor* k,
                                        const tl_hip_tensor* v, int64_t pos0, float scale);

/* ------------------------------------------------------ Llama decoder driver ----- */
/* The model composition of examples/apps/tinyllama/chatbot.tl:1-226 (Linear / RMSNorm /
 * MLP / Attention / Block and the decode loop), run on the device with a persistent f16 KV
 * cache in place of cat_4d + KVCache.update (system.rs:387-600).  Weight slots: which =
 * 0 attn_q, 1 attn_k, 2 attn_v, 3 attn_output, 4 ffn_gate, 5 ffn_up, 6 ffn_down; layer -1
 * is the LM head ("output.weight"); norms: which 0 attn_norm, 1 ffn_norm, layer -1
 * output_norm. */
tl_hip_llama* tl_hip_llama_new(int n_layers, int d_model, int n_heads, int n_kv_heads,
                               int ffn_dim, int vocab, float eps, float rope_theta,
                               int max_seq);
int tl_hip_llama_free(tl_hip_llama* m);
int tl_hip_llama_set_linear(tl_hip_llama* m, int layer, int which, int ggml_type,
                            const uint8_t* data, size_t nbytes);
int tl_hip_llama_set_norm(tl_hip_llama* m, int layer, int which, const float* w);
int tl_hip_llama_set_embedding(tl_hip_llama* m, const float* table);
/* Every weight of the decoder from a GGUF tensor map under the names chatbot.tl reads
 * (Block::from_map / Attention / MLP / RMSNorm::new, chatbot.tl:10-26, 44-47, 94-99, and
 * token_embd / output_norm / output, 153-155): blk.{i}.attn_{q,k,v,output}.weight,
 * blk.{i}.ffn_{gate,up,down}.weight, blk.{i}.{attn,ffn}_norm.weight.  Shapes are checked
 * against the decoder's configuration. */
int tl_hip_llama_load_gguf(tl_hip_llama* m, tl_hip_gguf* g);
/* KV-cache element type (kv_f16: 0 = f32, the tl_cpu cache; 1 = f16) and RoPE position rule
 * (rope_per_token: 0 = tl_cpu's, every token of a call rotated by the table row of the call's
 * start position, chatbot.tl:56-61 + ffi.rs:2655-2681; 1 = token t at start + t).  Resets the
 * cache. */
int tl_hip_llama_configure(tl_hip_llama* m, int kv_f16, int rope_per_token);
/* Whether the decoder's f16 prefill applies RoPE and the KV-cache append in the epilogue of
 * the [q | k | v] projection GEMM (default 1) or in a separate kernel after a plain GEMM (0);
 * the same values either way.  Returns the previous setting; on < 0 changes nothing and
 * returns the current one.  Instrumentation for the parity tests, which run both forms; no
 * reference counterpart. */
int tl_hip_debug_prefill_rope_epilogue(int on);
/* KVCache::new / free (system.rs:387-454): empties the cache. */
int tl_hip_llama_reset(tl_hip_llama* m);
/* Number of cached positions (the chatbot's start_pos for the next call). */
int64_t tl_hip_llama_position(const tl_hip_llama* m);
/* Number of hipGraph captures of the decode step so far (instrumentation; no reference
 * counterpart).  Two graphs are kept, one step and eight consecutive steps, each captured
 * the first time a graph decode needs it and again after a change of weights, configuration
 * or penalty value. */
int64_t tl_hip_llama_graph_builds(const tl_hip_llama* m);
/* One pass of the decode-loop body (chatbot.tl:174-187) over n new token ids at the
 * current cache position; writes the last row's logits [vocab] to logits_out (host,
 * may be NULL). prefill_f16 selects the f16-MFMA GEMM for the n > 4 linears. */
int tl_hip_llama_forward(tl_hip_llama* m, const int32_t* ids, int n, float* logits_out,
                         int prefill_f16);
/* Greedy choice from the logits of the last forward call, on the device:
 * repetition_penalty(history, p) (device_impl.rs:967-1001) then sample(temp <= 0) = argmax
 * (tensor.rs:1633-1637); returns the token id or -1 on error. */
int32_t tl_hip_llama_sample_greedy(tl_hip_llama* m, double repetition_penalty,
                                   const int32_t* history, int n_history);
/* The next token from the logits of the last forward call as chatbot.tl:188-189 takes it:
 * repetition_penalty(history, p), then sample(temp, top_p) (tensor.rs:1626-1680) with this
 * library's per-thread uniform draw (tl_hip_sample_seed).  temp <= 0: as
 * tl_hip_llama_sample_greedy.  Returns the token id or -1 on error. */
int32_t tl_hip_llama_sample(tl_hip_llama* m, float temp, float top_p, double repetition_penalty,
                            const int32_t* history, int n_history);
/* How tl_hip_llama_generate chooses each token: temp <= 0 (the default) greedy; otherwise
 * sample(temp, top_p) of the penalised logits, one uniform draw per step from the calling
 * thread's generator, drawn in step order before the steps run.  NaN values are
 * ArgumentError. */
int tl_hip_llama_set_sampling(tl_hip_llama* m, float temp, float top_p);
/* Decode of n_steps tokens after the cached context (chatbot.tl:174-222), each token chosen
 * as tl_hip_llama_set_sampling says (greedy by default): first token id `first`, generated
 * ids to out_ids (host).  repetition_penalty 1.0 disables the penalty; history holds the
 * prior ids (host). With use_graph != 0 the steps are captured hipGraph replays: one launch
 * per eight steps, then one per remaining step.  Both graph shapes (one step, eight steps)
 * are captured on the first graph-mode call after a change of penalty value, KV type, RoPE
 * mode or sampling settings, whatever its n_steps, so later calls only replay. */
int tl_hip_llama_generate(tl_hip_llama* m, int32_t first, int n_steps, int32_t* out_ids,
                          double repetition_penalty, const int32_t* history, int n_history,
                          int use_graph);

#ifdef __cplusplus
}
#endif
#endif /* TL_HIP_H */
