/*
 * scunet_hip.h - the C ABI of the MI355X SCUNet backend (libscunet_hip.so).
 *
 * This is the drop-in boundary for the reference crate's `--device gpu` path
 * (jacobsparts/scunet-rs). Every entry point below states which reference
 * interface it replaces. Plain pointers and sizes only; no HIP or torch types
 * appear in any signature, so a Rust `extern "C"` block, ctypes, or any other FFI
 * binds it directly.
 *
 * Conventions
 *   - Status: 0 = OK. Non-zero = the reference's `Err(String)`; the message is
 *     available from scunet_hip_last_error(handle) (or scunet_hip_create_error()
 *     when there is no handle yet). Nothing here aborts on a device error or OOM.
 *   - Planes are NCHW float32 `[c][h][w]`, the layout of Backend::forward.
 *   - One handle per thread (the reference's `Cuda` is `&mut self`, not Sync). A
 *     handle owns one HIP stream, created at default priority; every launch and
 *     copy of that handle is ordered on it.
 *   - "_device" entry points take device pointers, are stream-ordered on the
 *     handle's stream and do not synchronize; everything else takes host pointers
 *     and returns after the result is on the host.
 */
#ifndef SCUNET_HIP_H
#define SCUNET_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct scunet_hip scunet_hip;

/* Stage hook: called with one of the 16 stage names of cpu.rs:1175-1321
 * ("m_head", "m_down1_blocks", "m_down1", ..., "m_tail_in", "m_tail") and that
 * stage's plane as NCHW host floats (n elements), valid only during the call. */
typedef void (*scunet_stage_hook)(const char* name, const float* plane, size_t n, void* user);

/* --- construction (src/cuda.rs:192-241 Cuda::new, src/weights.rs:101-185 Weights::load) --- */

/* Load a SCUNet safetensors checkpoint, validate its __metadata__ keys and every
 * tensor shape exactly as weights.rs:204-280 does, and upload (repacked) to the
 * device. Fails with a message naming the field or tensor. */
int scunet_hip_create(const char* safetensors_path, scunet_hip** out);
/* The architecture of a checkpoint the caller has already loaded: the fields of the
 * reference's `Weights` (src/weights.rs:83-97): arch.name(), in_nc, dim, head_dim, window,
 * config ([down1, down2, down3, body, up3, up2, up1]). */
typedef struct {
    const char* variant;
    size_t in_nc, dim, head_dim, window;
    size_t config[7];
} scunet_hip_arch_info;

/* Weights::t / shape (src/weights.rs:312-320) as a callback: return the float32 data of
 * tensor `name` (row-major) and write its shape to shape[0..*ndim) (at most 8 extents),
 * or return NULL when there is no such tensor. The data is read during the create call
 * only. */
typedef const float* (*scunet_hip_tensor_lookup)(void* user, const char* name, size_t* shape,
                                                 size_t* ndim);

/* Cuda::new(&'a Weights) (src/cuda.rs:192-241) on tensors the caller has already loaded:
 * every tensor the network uses is requested by name through `lookup`, validated
 * exactly as scunet_hip_create validates a file (weights.rs:204-280: a missing tensor or
 * a wrong shape fails with the same message, the file path replaced by "weights"), and
 * uploaded. No file is read, so a checkpoint the caller mmapped is loaded once. */
int scunet_hip_create_from_tensors(const scunet_hip_arch_info* arch, scunet_hip_tensor_lookup lookup,
                                   void* user, scunet_hip** out);
/* Message of the last failed scunet_hip_create or scunet_hip_create_from_tensors on this
 * thread. */
const char* scunet_hip_create_error(void);
void scunet_hip_destroy(scunet_hip* h);
/* Message of the last failed call on this handle ("" if none). */
const char* scunet_hip_last_error(const scunet_hip* h);

/* Backend::name (src/backend.rs:20-21): "hip". */
const char* scunet_hip_name(const scunet_hip* h);
/* The architecture read from the checkpoint (weights.rs:84-98). config has 7 entries. */
int scunet_hip_arch(const scunet_hip* h, int* in_nc, int* dim, int* head_dim, int* window,
                    int* config);
/* The checkpoint's variant, one of the eight published names (Weights::arch.name(),
 * weights.rs:62-73), e.g. "color-real-psnr"; "" for a null handle. */
const char* scunet_hip_variant(const scunet_hip* h);

/* --- arithmetic mode (no counterpart in the reference, whose GPU path is fp32 only) ---
 * SCUNET_HIP_FP32 (the default): fp32 operands, planes and accumulation, the reference's
 * arithmetic to fp32 rounding. Where a kernel has the form, a matrix product runs on the
 * bf16 matrix cores from an exact three-way bf16 split of each fp32 operand (x = h + m + l
 * exactly) as the six part products that can exceed 2^-24 |ab|, accumulated in fp32; the
 * three dropped are below 2^-25 |ab| together, less than fp32's own rounding of one
 * product. The other products run on the fp32 matrix cores.
 * SCUNET_HIP_FP32_MFMA: every product on the fp32 matrix cores (v_mfma_f32_16x16x4_f32).
 * SCUNET_HIP_FP16: the matrix products take fp16 operands (round to nearest even) with fp32
 * accumulation; planes, residuals, LayerNorm, softmax and GELU stay fp32. Faster, and
 * within a stated looser tolerance of the fp32 result (max abs error and PSNR against
 * the fp32 output are part of the test suite and the benchmark report).
 * The mode applies to the handle's following calls. */
#define SCUNET_HIP_FP32 0
#define SCUNET_HIP_FP16 1
#define SCUNET_HIP_FP32_MFMA 2
int scunet_hip_set_precision(scunet_hip* h, int mode);
/* The handle's mode, or -1 for a null handle. */
int scunet_hip_precision(const scunet_hip* h);

/* --- the forward (src/backend.rs:23-25 Backend::forward; src/cuda.rs:1606-1848) --- */

/* x: the already replicate-padded plane [c][hp][wp] (hp, wp multiples of 64, c = in_nc);
 * y: caller-allocated [c][hp][wp]. */
int scunet_hip_forward(scunet_hip* h, const float* x, size_t c, size_t hp, size_t wp, float* y);
/* Same contract on device pointers, stream-ordered, no synchronization. */
int scunet_hip_forward_device(scunet_hip* h, const float* x, size_t c, size_t hp, size_t wp,
                              float* y);
/* forward with the stage hook of cpu.rs:1175-1321 (forward_dump). */
int scunet_hip_forward_dump(scunet_hip* h, const float* x, size_t c, size_t hp, size_t wp,
                            float* y, scunet_stage_hook hook, void* user);

/* --- pad, forward, crop (src/backend.rs:63-105 backend::run; plan.rs:67-94) ---
 * x: the image [c][hh][ww] in [0,1], any size; y: [c][hh][ww]. The replicate pad to
 * ceil64 and the crop happen on the device, fused into the first and last convolution.
 * Fails like plan.rs:105-118 check_min_size. */
int scunet_hip_run(scunet_hip* h, const float* x, size_t c, size_t hh, size_t ww, float* y);
int scunet_hip_run_device(scunet_hip* h, const float* x, size_t c, size_t hh, size_t ww, float* y);

/* scunet_hip_run_device for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in
 * the reference. Same arguments and result as scunet_hip_run_device (device pointers,
 * stream-ordered on the handle's stream), but the forward's scratch is a static device
 * array of 256 MiB per GPU, which the library holds from the first handle created on that
 * GPU until the process ends: no hipMalloc, hipFree or other allocation happens in the
 * call. Limit: the padded image needs 1600 bytes of scratch per pixel (plus 256-byte
 * alignment per role), so padded planes up to about 167 000 pixels fit (384x384, 512x320);
 * a larger image fails with an error naming both sizes. Every call on one GPU shares
 * that GPU's array: calls that overlap in time on one GPU (two handles, two threads or
 * streams) race and corrupt each other's results; serialise them. Profiling events are
 * not recorded during the call. */
int scunet_hip_run_device_noalloc(scunet_hip* h, const float* x, size_t c, size_t hh, size_t ww,
                                  float* y);

/* n images of one size, [n][c][hh][ww] in and out, host buffers (backend::run,
 * backend.rs:63-105, over a batch): one upload, one forward over the n padded images stacked
 * along y as one plane (every kernel keeps each image's edges as plane edges, so each
 * result is bit-identical to the image's own forward), one download. Many small images then
 * fill the device as one large one does. */
int scunet_hip_run_batch(scunet_hip* h, const float* x, size_t n, size_t c, size_t hh, size_t ww, float* y);

/* --- will it fit (src/memguard.rs:66-74 device_need; 1-80 for the policy) ---
 * The device memory a forward of an hh x ww image (padded to ceil64 on each axis) takes,
 * computed from the scratch roles the forward requests rather than fitted:
 * *scratch_bytes = the handle's scratch arena after such a forward (the arena keeps each
 * role's largest size), *more_bytes = what it does not hold yet. host_io != 0 counts the
 * host entry points' staging copies of x and y. Weights are not included (footprint).
 * Every forward entry point asks this before its first allocation and, when *more_bytes
 * exceeds the device's free memory, fails with a message naming the sizes instead of
 * failing in an allocation. */
int scunet_hip_device_need(const scunet_hip* h, size_t c, size_t hh, size_t ww, int host_io,
                           size_t* scratch_bytes, size_t* more_bytes);

/* --- Backend's bookkeeping (src/backend.rs:30-55) --- */
int scunet_hip_footprint(const scunet_hip* h, size_t* weight_bytes, size_t* scratch_bytes);
int scunet_hip_release_scratch(scunet_hip* h);
int scunet_hip_synchronize(scunet_hip* h);
/* The handle's hipStream_t, as void*. */
void* scunet_hip_stream(scunet_hip* h);

/* Per-launch device timing (the SCUNET_PROFILE instrument of cuda.rs:106-135, 263-273,
 * 1875-1884): when on, every launch is bracketed by a pair of HIP events on the
 * handle's stream. profile_report synchronizes and fills up to `cap` rows of
 * (kernel-class name, launches, total ms, algorithmic FLOP, algorithmic bytes), sorted
 * by total time; returns the number of classes in *n. Names stay valid until the next
 * profile call on the handle. */
int scunet_hip_profile(scunet_hip* h, int on);
int scunet_hip_profile_report(scunet_hip* h, const char** names, long* launches, double* ms,
                              double* flop, double* bytes, int cap, int* n);

/* --- device memory for callers without a device allocator (tests, bench) --- */
int scunet_hip_malloc(scunet_hip* h, void** p, size_t bytes);
int scunet_hip_free(scunet_hip* h, void* p);
int scunet_hip_h2d(scunet_hip* h, void* dst, const void* src, size_t bytes);
int scunet_hip_d2h(scunet_hip* h, void* dst, const void* src, size_t bytes);

/* A plain streaming device-to-device copy kernel on the handle's stream (no counterpart
 * in the reference): the known-size kernel that hardware traffic counters are
 * calibrated against. bytes must be a multiple of 16 and both pointers 16-byte aligned. */
int scunet_hip_copy(scunet_hip* h, void* dst, const void* src, size_t bytes);

/* --- probes (src/cuda.rs:1153-1597), host buffers in the reference's layouts --- */

/* Cuda::block_dump (cuda.rs:1153-1167): one ConvTransBlock `prefix` on x [c][hh][ww]. */
int scunet_hip_block_probe(scunet_hip* h, const char* prefix, size_t hh, size_t ww, size_t shift,
                           const float* x, float* out);
/* Cuda::op_probe (cuda.rs:1173-1202): op in {"conv3x3", "conv1x1", "conv2x2s2",
 * "conv_t2x2"} with weight `name` (+".weight", and ".bias" when present) on x
 * [c_in][hh][ww]; out is [c_out][hh][ww] (conv2x2s2: [c_out][hh/2][ww/2], conv_t2x2:
 * [c_out][2hh][2ww]). */
int scunet_hip_op_probe(scunet_hip* h, const char* op, const char* name, const float* x,
                        size_t c_in, size_t c_out, size_t hh, size_t ww, float* out);
/* Cuda::linear_probe (cuda.rs:1471-1481): x [rows][c_in] -> out [rows][c_out]. */
int scunet_hip_linear_probe(scunet_hip* h, const char* name, const float* x, size_t rows,
                            size_t c_in, size_t c_out, float* out);
/* Cuda::layer_norm_probe (cuda.rs:1484-1494): x [rows][c] -> out [rows][c]. */
int scunet_hip_layer_norm_probe(scunet_hip* h, const char* name, const float* x, size_t rows,
                                size_t c, float* out);
/* Cuda::attention_kernel_probe (cuda.rs:1501-1519): the attention core alone on window-
 * major qkv [nw*64][3c] (q | k | v column blocks, head j = columns j*hd..j*hd+hd-1 of
 * each) with rel-pos table rp [heads][15][15]; out [nw*64][c]. The window grid is
 * (hh/8) x (ww/8); shift > 0 applies the shifted-window mask. */
int scunet_hip_attention_kernel_probe(scunet_hip* h, size_t hh, size_t ww, size_t c, size_t heads,
                                      size_t hd, size_t shift, const float* qkv, const float* rp,
                                      float* out);
/* Cuda::gather_probe (cuda.rs:1523-1537): the window index map the attention kernel
 * uses, x [c][hh][ww] -> tokens [nw*64][c]. */
int scunet_hip_gather_probe(scunet_hip* h, size_t hh, size_t ww, size_t c, size_t shift,
                            const float* x, float* tok);
/* Cuda::window_round_trip (cuda.rs:1543-1560): gather then scatter, x -> out. */
int scunet_hip_window_round_trip(scunet_hip* h, size_t hh, size_t ww, size_t c, size_t shift,
                                 const float* x, float* out);
/* Cuda::attention_probe (cuda.rs:1569-1597): gather + LN1 + qkv + attention + proj of
 * block `prefix` on x [c][hh][ww]; returns the token buffer [nw*64][c] in window order. */
int scunet_hip_attention_probe(scunet_hip* h, const char* prefix, size_t hh, size_t ww, size_t c,
                               size_t shift, const float* x, float* tok);

/* Cuda::bench_attn (cuda.rs:1438-1468) on device buffers: the attention core over
 * window-major qkv [nwh*nww*64][3c] -> out [nwh*nww*64][c], rp [heads][15][15] on the
 * host. Runs 3 warmups then `iters` launches, timed with HIP events on the handle's
 * stream; *ms = mean device time per launch. */
int scunet_hip_bench_attn(scunet_hip* h, const float* qkv, const float* rp, float* out, size_t nwh,
                          size_t nww, size_t c, size_t heads, size_t shift, int iters, double* ms);

#ifdef __cplusplus
}
#endif

#endif /* SCUNET_HIP_H */
