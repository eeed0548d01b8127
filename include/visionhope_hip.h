/*
 * visionhope_hip.h — C ABI of libvisionhope_hip.so, the MI355X (gfx950) kernels
 * for VisionHOPE's SRNL operator hot path.
 *
 * Conventions shared by every entry point:
 *   - All tensor arguments are raw device pointers to dense (contiguous) memory
 *     in the layout stated next to each argument; sizes are int64_t.
 *   - `stream` is a hipStream_t passed as void*.  Work is enqueued on it
 *     asynchronously; nothing synchronises, allocates or frees device memory,
 *     so every call can be recorded into a HIP graph.
 *   - The caller owns every buffer: outputs and workspaces are allocated by the
 *     caller (workspace sizes come from the *_workspace_bytes queries).
 *   - Return value: VH_OK (0) or one of the VH_ERR_* codes below; a message for
 *     the last failure on the calling thread is available from vh_last_error().
 *   - io_dtype selects the element type of activation tensors (x, q, y):
 *     VH_DTYPE_F32, VH_DTYPE_BF16 or VH_DTYPE_F16.  SRNL memories, skips,
 *     weights and fused outputs are always fp32, as in the reference.
 *
 * Each declaration cites the reference interface it replaces (path:line inside
 * the PSRben/VisionHOPE repository).
 */
#ifndef VISIONHOPE_HIP_H
#define VISIONHOPE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VH_ABI_VERSION 1

enum {
    VH_OK = 0,
    VH_ERR_SHAPE = 1,      /* inconsistent or empty shapes */
    VH_ERR_DTYPE = 2,      /* unsupported element type */
    VH_ERR_HEAD_DIM = 3,   /* head_dim not in {4, 8, 16, 32, 64} */
    VH_ERR_WORKSPACE = 4,  /* workspace missing or too small */
    VH_ERR_ARG = 5,        /* null pointer or out-of-range scalar */
    VH_ERR_LAUNCH = 6      /* the HIP runtime rejected a launch */
};

enum { VH_DTYPE_F32 = 0, VH_DTYPE_BF16 = 1, VH_DTYPE_F16 = 2 };

/* Stability constants of the recurrence.  Replaces the text substitution of
 * __ETA_SCALE__ ... __ETA2ALPHA_FACTOR__ into the CUDA sources
 * (models/srnl_core/chunk.py:44-49,89-97; fused.py:38-49): here they are
 * run-time arguments instead of compile-time literals. */
typedef struct vh_srnl_consts {
    float step_scale;        /* ETA_SCALE        = VISIONHOPE_STEP_SCALE (0.025) */
    float min_retention;     /* ALPHA_MIN        = VISIONHOPE_MIN_RETENTION (0) */
    float retention_bias;    /* ALPHA_BIAS       = VISIONHOPE_RETENTION_BIAS (ln 9) */
    float injection_margin;  /* STAB_MU          = VISIONHOPE_INJECTION_MARGIN (0.999) */
    int32_t spectral_clamp;  /* ETA2ALPHA_CLAMP  = SPECTRAL_CLAMP (1) */
    float spectral_factor;   /* ETA2ALPHA_FACTOR = 2 * VISIONHOPE_SPECTRAL_MARGIN */
} vh_srnl_consts;

int vh_abi_version(void);
const char* vh_last_error(void);

/* Dispatch overrides, for tests and measurements only.  No counterpart in the
 * reference (its only environment reads are the numerics constants,
 * models/srnl_core/chunk.py:34-58).  Every entry point chooses its kernel
 * variant from its own arguments; nothing is read from the environment.
 * vh_set_dispatch_override(name, value) forces one choice for every later call
 * in this process until it is cleared (value NULL or ""); an unknown name or a
 * malformed value returns VH_ERR_ARG and changes nothing.  Names and values:
 *   scan_ut          "0" | "1"        SRNL head_dim 16 and 32: stepped form / block form
 *   scan_wide        "0"|"1"|"2"|"4"  SRNL: waves per line of the wide scan (0: none)
 *   scan_tb          "1" | "2"        wide scan: row split / token blocks
 *   scan_pack        "<L>x<T>"        head_dim-16 scans: lines and 16-slot tiles per wave
 *   scan_utw         "0" | "1"        head_dim 16 and 32: the block form with a chunk's
 *                                     blocks over the waves of one workgroup per line, never /
 *                                     whenever the chunks allow (default: head_dim 16 below
 *                                     1024 lines; head_dim 32 always, chunks up to 64)
 *   pw_cfg, pw_resident               1x1 convolution kernel variants
 *   dw_tile, dw_tile_cs, dw_tile_p, dw_launch_bytes   depthwise kernel variants
 *   ln_stage         "0" | "1"        LayerNorm staged stores
 *   conv_band        "0" | "1"        3x3 convolution band kernel
 *   grn_spin_limit   1 .. 2^20        one-pass GRN: sleeps before a piece stops waiting
 *                                     for the other pieces of its image
 *   fusion_tile      "<a>x<b>x<h>"    direction fusion: 2^a x 2^b pixel tiles, h heads per
 *                                     workgroup
 *   grn_pieces       2 .. 64          one-pass GRN: pieces per image
 *   readout_tile     "8" | "16"       SRNL tile readout: pixel tile edge (default 8 for maps
 *                                     of at most 8 x 8, else 16)
 * Results stay within each kernel's stated tolerance under every override: an
 * override changes which kernel runs, never what it computes. */
int vh_set_dispatch_override(const char* name, const char* value);
void vh_clear_dispatch_overrides(void);

/* ---------------------------------------------------------------------------
 * SRNL recurrence.  Every SRNL entry point runs the same two kernels: a scan
 * over the chunks of each (batch, direction, head) line that writes the
 * chunk-start content memory of every chunk into the workspace, and a readout
 * that computes y = M_m^chunk q_hat for every token (and, for the spatial
 * entries, restores and fuses the four directions).
 * Memories: M_m/M_v/M_k [R, heads, d, d], M_eta/M_alpha [R, heads, d], fp32,
 * shared over the batch (chunk.py:193-196).
 * ------------------------------------------------------------------------- */

/* Workspace for the chunk-start content memories of `lines` lines whose
 * longest scan has `max_chunks` chunks of head_dim x head_dim fp32. */
size_t vh_srnl_workspace_bytes(int64_t lines, int64_t max_chunks, int32_t head_dim);

/* Four-direction spatial operator on channels-last activations: x and q are
 * [B, H, W, C] (q = W_q x + b, computed once per token), out is [B, H, W, C]
 * fp32 = sum_r dir_weight[r, c] * (y_r + d_skip[r, c] * x).  chunks[r] is the
 * chunk length of scan r ((W, W, H, H) on the spatial path).
 * d_skip holds C values (skip_per_direction = 0) or 4*C values (= 1).
 * Workspace: vh_srnl_workspace_bytes(B*4*heads, max_r ceil(H*W/chunks[r]), d).
 * Replaces VisionHOPEOperator._forward_fast's serialize/stack + the fused
 * kernel call (models/operator.py:172-193, models/srnl_core/csrc/fused.cu:307-351)
 * without materialising the four serialized copies of x and q. */
int vh_srnl_spatial_forward(
    const void* x, const void* q, int32_t io_dtype,
    const float* M_m, const float* M_v, const float* M_k,
    const float* M_eta, const float* M_alpha,
    const float* d_skip, int32_t skip_per_direction, const float* dir_weight,
    float* out, int64_t B, int64_t H, int64_t W, int64_t C, int32_t head_dim,
    const int64_t chunks[4], const vh_srnl_consts* consts,
    void* workspace, size_t workspace_bytes, void* stream);

/* vh_srnl_spatial_forward without a workspace argument: the chunk-start memories go to
 * a fixed 96 MiB device array of the library (one per GPU, held from the first call on that
 * GPU until the process ends), so the call allocates nothing.  No counterpart in the
 * reference; it is for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc).  A call whose
 * vh_srnl_workspace_bytes exceeds 96 MiB returns VH_ERR_WORKSPACE.  Calls that overlap on
 * one GPU (several streams or host threads) share the array and race. */
int vh_srnl_spatial_forward_noalloc(
    const void* x, const void* q, int32_t io_dtype,
    const float* M_m, const float* M_v, const float* M_k,
    const float* M_eta, const float* M_alpha,
    const float* d_skip, int32_t skip_per_direction, const float* dir_weight,
    float* out, int64_t B, int64_t H, int64_t W, int64_t C, int32_t head_dim,
    const int64_t chunks[4], const vh_srnl_consts* consts, void* stream);

/* The two halves of vh_srnl_spatial_forward, for callers that overlap other work with
 * the scan (the readout needs q; the scan does not).  vh_srnl_spatial_scan writes the
 * chunk-start memories of every line into the workspace; vh_srnl_spatial_readout reads
 * them (same workspace, same chunks, ordered after the scan) and writes out [B, H, W, C]
 * = sum_r dir_weight[r, c] (y_r + d_skip[r, c] x) + aux, with aux an optional io-dtype
 * [B, H, W, C] addend (NULL: none) and out stored as out_dtype (fp32 or io_dtype).  No
 * counterpart in the reference (its fused kernel does both, fused.cu:307-351); the
 * prepared block uses aux for the local position encoding (models/block.py:77-78).
 * The workspace contents are private to the pair: for bf16 maps with head_dim 16 and at
 * least 1024 lines (B*4*heads) each 16-byte slot of a state holds four entries as bf16
 * hi then lo halves (the same size as FP32), otherwise FP32. */
int vh_srnl_spatial_scan(
    const void* x, int32_t io_dtype, const float* M_m, const float* M_v, const float* M_k,
    const float* M_eta, const float* M_alpha, int64_t B, int64_t H, int64_t W, int64_t C,
    int32_t head_dim, const int64_t chunks[4], const vh_srnl_consts* consts,
    void* workspace, size_t workspace_bytes, void* stream);
int vh_srnl_spatial_readout(
    const void* x, const void* q, int32_t io_dtype, const float* d_skip, int32_t skip_per_direction,
    const float* dir_weight, const void* aux, void* out, int32_t out_dtype, int64_t B, int64_t H,
    int64_t W, int64_t C, int32_t head_dim, const int64_t chunks[4], const void* workspace,
    size_t workspace_bytes, void* stream);
/* vh_srnl_spatial_readout with the block's local position encoding computed in the same
 * pass: out (io dtype) = the readout + io_dtype(conv5x5(x) + lepe_bias), conv5x5 the
 * depthwise 5x5 convolution of x with zero padding, lepe_taps [25, C] FP32 taps-major
 * (tap dy*5+dx of channel c at [dy*5+dx][c]) and lepe_bias [C] FP32 or NULL.  The same
 * bits as vh_dwconv2d_nhwc_forward (ksize 5, plain epilogue) followed by
 * vh_srnl_spatial_readout with that result as aux and out_dtype = io_dtype.  No
 * counterpart in the reference, whose block adds local_position(x_local) to the operator
 * output in a separate step (models/block.py:77-78). */
int vh_srnl_spatial_readout_lepe(
    const void* x, const void* q, int32_t io_dtype, const float* d_skip, int32_t skip_per_direction,
    const float* dir_weight, const float* lepe_taps, const float* lepe_bias, void* out, int64_t B,
    int64_t H, int64_t W, int64_t C, int32_t head_dim, const int64_t chunks[4], const void* workspace,
    size_t workspace_bytes, void* stream);

/* Backward of the packed SRNL forward: vh_srnl_sequence_forward (q_raw = 1, q [B, R, N,
 * heads*d] in io_dtype) or vh_srnl_forward (q_raw = 0, pre-normalised fp32 q [B, R, heads,
 * N, d]), with the same x, memories, memories_per_line and chunks.  dy [B, R, heads, N, d]
 * fp32 is the gradient of y; outputs fp32: dx like x, dq like q, and the gradients of the
 * five initial memories (summed over the batch when shared).  Chunks in [1, 64], head_dim
 * 4, 8, 16 or 32; workspace from vh_srnl_backward_workspace_bytes.  Replaces
 * srnl_backward / srnl_backward_qraw (models/srnl_core/csrc/chunk.cu:511-1057, bound at
 * chunk.py:289-359 and 510-588); the forward is recomputed from the inputs instead of
 * read from tensors saved by a training forward. */
size_t vh_srnl_backward_workspace_bytes(int64_t B, int64_t R, int64_t heads, int64_t N, int32_t head_dim,
                                        const int64_t* chunks);
int vh_srnl_backward(
    const void* x, const void* q, int32_t io_dtype, int32_t q_raw, const float* dy,
    const float* M_m, const float* M_v, const float* M_k, const float* M_eta, const float* M_alpha,
    int32_t memories_per_line, float* dx, float* dq, float* dM_m, float* dM_v, float* dM_k, float* dM_eta,
    float* dM_alpha, int64_t B, int64_t R, int64_t heads, int64_t N, int32_t head_dim, const int64_t* chunks,
    const vh_srnl_consts* consts, void* workspace, size_t workspace_bytes, void* stream);

/* The reference's fused spatial entry with its own argument layout: X and
 * Q_raw are the serialized stacks [B, 4, H*W, C]; Out is [B, H, W, C] fp32;
 * chunks are (W, W, H, H).  Replaces srnl_line_forward_seq_noatomic
 * (models/srnl_core/csrc/fused.cu:307-351, bound at fused.py:70-76). */
int vh_srnl_line_forward_seq_noatomic(
    const void* X, const void* Q_raw, int32_t io_dtype,
    const float* M_m, const float* M_v, const float* M_k,
    const float* M_eta, const float* M_alpha,
    const float* d_skip, int32_t skip_per_direction, const float* dir_weight,
    float* out, int64_t B, int64_t H, int64_t W, int64_t C, int32_t head_dim,
    const vh_srnl_consts* consts, void* workspace, size_t workspace_bytes, void* stream);

/* Packed sequences: X [B, R, heads, N, d], Q_raw [B, R, N, heads*d] (raw,
 * normalised per head inside), Out [B, R, heads, N, d] in io_dtype; chunks[r]
 * per direction (R in {1, 2, 4}); the final chunk is zero-padded.
 * memories_per_line = 1: the memories hold one state per line, shaped
 * [B*R*heads, d, d] / [B*R*heads, d] (the reference's 5-D memories,
 * chunk.py:193-198, chunk.cu:287).
 * Workspace: vh_srnl_workspace_bytes(B*R*heads, max_r ceil(N/chunks[r]), d).
 * Replaces srnl_sequence_forward (models/srnl_core/csrc/fused.cu:131-179) and
 * the forward halves of srnl_forward_qraw (chunk.cu:1106-1131),
 * srnl_forward_qraw_large / _varline (lines.cu:688-732). */
int vh_srnl_sequence_forward(
    const void* X, const void* Q_raw, int32_t io_dtype,
    const float* M_m, const float* M_v, const float* M_k,
    const float* M_eta, const float* M_alpha, int32_t memories_per_line,
    void* out, int64_t B, int64_t R, int64_t heads, int64_t N, int32_t head_dim,
    const int64_t* chunks, const vh_srnl_consts* consts,
    void* workspace, size_t workspace_bytes, void* stream);

/* Packed sequences with pre-normalised fp32 queries Q [B, R, heads, N, d]
 * (used as given).  Replaces the forward half of srnl_forward
 * (models/srnl_core/csrc/chunk.cu:1083-1104, called at chunk.py:234). */
int vh_srnl_forward(
    const void* X, int32_t io_dtype, const float* Q,
    const float* M_m, const float* M_v, const float* M_k,
    const float* M_eta, const float* M_alpha, int32_t memories_per_line,
    void* out, int64_t B, int64_t R, int64_t heads, int64_t N, int32_t head_dim,
    const int64_t* chunks, const vh_srnl_consts* consts,
    void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Elementwise tail
 * ------------------------------------------------------------------------- */

/* Direction fusion: Y, X [B, 4, heads, H*W, d] (io_dtype) ->
 * out [B, C, H, W] fp32 = sum_r scale[r, c] * (y_r + d_skip[r, c] * x_r),
 * restored to image order; channels_last selects NHWC storage of out.
 * Replaces visionhope_postprocess_scale_forward
 * (utils/csrc/direction_fusion.cu:505-575, called at direction_fusion.py:95). */
int vh_postprocess_scale_forward(
    const void* Y, const void* X, int32_t io_dtype,
    const float* d_skip, int32_t skip_per_direction, const float* scale,
    float* out, int64_t B, int64_t heads, int64_t H, int64_t W, int32_t head_dim,
    int32_t channels_last, void* stream);

/* Workspace of vh_grn_forward and vh_grn_scale_forward: a 32 KiB header of
 * synchronisation words, then B * pieces * C fp32 partial sums.
 * The synchronisation words must be zero when a workspace is first used (zero the whole
 * workspace once); every call leaves them zero, so the workspace can be reused as is.
 * Calls that share a workspace must not overlap (use one workspace per stream). */
size_t vh_grn_workspace_bytes(int64_t B, int64_t C, int64_t H, int64_t W);

/* Diagnostic, not for graph capture: synchronises `stream`, then sets *count to the
 * number of times a workgroup of vh_grn_forward's one-pass kernel on this workspace
 * stopped waiting for the other workgroups of its image and computed the image's
 * statistics from x itself (its output is still correct; the count only shows that
 * the wait gave up).  The count is never reset by the library.  No counterpart in
 * the reference, whose GRN has no cross-workgroup wait (grn_cuda.cu:290-320). */
int vh_grn_workspace_fallbacks(const void* workspace, size_t workspace_bytes, void* stream, int64_t* count);

/* Whether `stream` is capturing a HIP graph and, if so, the capture's identifier (unique
 * per capture; *id = 0 otherwise).  A query that records nothing, valid during capture.
 * No counterpart in the reference: the GRN wrapper keeps one workspace per captured graph
 * (its zero fill a node of that graph) so that graphs replayed in any order never share
 * synchronisation words. */
int vh_stream_capture_id(void* stream, int32_t* capturing, uint64_t* id);

/* GRN on channels-last x [B, H, W, C] (io_dtype): gx = ||x||_2 over H*W,
 * nx = gx / (mean_c gx + eps), y = x (1 + gamma nx) + beta, y [B, H, W, C] computed
 * in fp32 and stored as y_dtype (VH_DTYPE_F32 reproduces the reference's output;
 * a 16-bit y_dtype stores what a following autocast cast would produce);
 * gx [B, C] and inv_den [B] are written too (the reference saves them for
 * backward).  Replaces grn_forward_cuda (utils/csrc/grn_cuda.cu:290-320,
 * called at utils/grn_cuda.py:42). */
int vh_grn_forward(
    const void* x, int32_t io_dtype, const float* gamma, const float* beta,
    void* y, int32_t y_dtype, float* gx, float* inv_den, int64_t B, int64_t C, int64_t H, int64_t W,
    float eps, void* workspace, size_t workspace_bytes, void* stream);

/* GRN statistics only, for consumers that apply GRN while loading its input
 * (vh_pointwise_conv_nhwc_forward): gx [B, C], inv_den [B] as vh_grn_forward, and
 * scale [B, C] = 1 + gamma * gx * inv_den, so that GRN(x) = x * scale + beta.
 * Channels-last x [B, H, W, C] (C % 8 == 0, C <= 2048, 16-byte aligned); same
 * workspace as vh_grn_forward.  Splits grn_forward_cuda
 * (utils/csrc/grn_cuda.cu:290-320) at its statistics/apply boundary. */
int vh_grn_scale_forward(
    const void* x, int32_t io_dtype, const float* gamma, float* gx, float* inv_den, float* scale,
    int64_t B, int64_t C, int64_t H, int64_t W, float eps, void* workspace,
    size_t workspace_bytes, void* stream);

/* LayerNorm over C for every pixel of x [B, C, H, W] (channels_last = 1: NHWC
 * storage, 0: NCHW storage), biased variance, y in the same storage order,
 * computed in fp32 and stored as y_dtype (VH_DTYPE_F32 is the reference's
 * output); mean/rstd [B*H*W] are optional (may be NULL).  Replaces the Triton
 * _layernorm2d_forward_kernel (utils/layer_norm_cuda.py:31-57,122-147) and the
 * F.layer_norm call of LayerNorm2d.inference_layout (models/layers.py:18-20). */
int vh_layernorm2d_forward(
    const void* x, int32_t io_dtype, const float* weight, const float* bias,
    void* y, int32_t y_dtype, float* mean, float* rstd, int64_t B, int64_t C, int64_t H, int64_t W,
    float eps, int32_t channels_last, void* stream);

/* Residual add followed by LayerNorm over C, on channels-last tensors: x_sum = x + r
 * rounded to io_dtype (written), y = LayerNorm(x_sum) computed in fp32 and stored as
 * y_dtype.  C % 8 == 0, 16-byte aligned tensors.  No counterpart in the reference's native
 * code: it fuses the residual add of VisionHOPEBlock.forward (models/block.py:105-106,
 * gamma folded by prepare_for_inference) with the following norm2 call. */
int vh_add_layernorm2d_forward(
    const void* x, const void* r, int32_t io_dtype, const float* weight, const float* bias,
    void* x_sum, void* y, int32_t y_dtype, int64_t B, int64_t C, int64_t H, int64_t W, float eps,
    void* stream);

/* Query normalisation + relayout: q_raw [B, R, N, heads*d] (io_dtype) ->
 * q [B, R, heads, N, d] fp32 = q_raw / max(||q_raw||, 1e-12) per head, and
 * inv_norm [B, R, heads, N].  Replaces visionhope_qnorm_forward
 * (utils/csrc/query_normalization.cu:223-265). */
int vh_qnorm_forward(
    const void* q_raw, int32_t io_dtype, float* q, float* inv_norm,
    int64_t B, int64_t R, int64_t N, int64_t heads, int32_t head_dim, void* stream);

/* Depthwise KxK convolution (K in {3, 5, 7}, stride 1, padding K/2) on a
 * channels-last x [B, H, W, C] (io_dtype, C % 8 == 0, 16-byte aligned tensors)
 * with taps [K*K, C] fp32 (taps-major) and bias [C] (or NULL), accumulated in
 * fp32, with the block's surrounding elementwise work fused:
 *   epilogue 0: out = conv(x) + b
 *   epilogue 1: out = x + conv(x) + b                      (block CPE)
 *   epilogue 2: out = x + sigmoid(aux) * (conv(x) + b)     (gated local conv)
 *   epilogue 3: out = gelu_erf(x + conv(x) + b)            (FFN dwconv + act)
 *   epilogue 4: out (fp32, in place) += conv(x) + b        (LePE into SRNL out)
 *   epilogue 5: out = aux + conv(x) + b, aux fp32          (LePE + SRNL out -> io dtype)
 * out/aux are [B, H, W, C] in io_dtype except the fp32 out of epilogue 4 and the fp32
 * aux of epilogue 5.  No counterpart in
 * the reference's native code: it runs PyTorch Conv2d plus separate
 * elementwise ops inside VisionHOPEBlock (models/block.py:63-107,
 * models/layers.py:73-77); this fuses them on the prepared inference path. */
int vh_dwconv2d_nhwc_forward(
    const void* x, int32_t io_dtype, const float* taps, const float* bias, int32_t ksize,
    int32_t epilogue, const void* aux, void* out, int64_t B, int64_t H, int64_t W, int64_t C,
    void* stream);

/* The block's CPE and the LayerNorm after it on a channels-last x [B, H, W, C]
 * (io_dtype): out = x + conv(x) + b as epilogue 1 of vh_dwconv2d_nhwc_forward
 * (ksize 3), and out_norm = LayerNorm over the C channels of out as stored, with
 * ln_weight / ln_bias [C] fp32 and eps, the bits that vh_layernorm2d_forward gives on
 * out (same reduction order).  C = 8 * 2^k <= 256; 16-byte aligned tensors.  No
 * counterpart in the reference's native code: it runs the CPE (a depthwise Conv2d plus
 * the residual add, models/block.py:102-103) and norm1 (LayerNorm2d,
 * models/block.py:104, utils/layer_norm_cuda.py) as separate modules; this fuses them
 * on the prepared inference path. */
int vh_dwconv2d_add_layernorm2d_forward(
    const void* x, int32_t io_dtype, const float* taps, const float* bias, int32_t ksize,
    const float* ln_weight, const float* ln_bias, float eps, void* out, void* out_norm,
    int64_t B, int64_t H, int64_t W, int64_t C, void* stream);

/* Workspace of vh_dwconv2d_gelu_grn_forward: B * (blocks per image) * C fp32 partial
 * sums, or 0 when the shape is not covered (C/8 must divide 256 and the kernel's
 * 256-thread blocks must tile whole images). */
size_t vh_dwconv2d_gelu_grn_workspace_bytes(int64_t B, int64_t H, int64_t W, int64_t C, int32_t ksize);

/* The FFN middle on a channels-last x [B, H, W, C] (io_dtype): out = gelu_erf(x +
 * conv(x) + b) as epilogue 3 of vh_dwconv2d_nhwc_forward, plus the GRN statistics of
 * out (as stored) from partial sums taken in the same pass: gx [B, C], inv_den [B] and
 * scale [B, C] = 1 + gamma * gx * inv_den as vh_grn_scale_forward gives them.  No
 * counterpart in the reference's native code (models/layers.py:73-77 runs the
 * depthwise conv, GELU and GRN as separate modules). */
int vh_dwconv2d_gelu_grn_forward(
    const void* x, int32_t io_dtype, const float* taps, const float* bias, int32_t ksize,
    const float* gamma, float eps, void* out, float* gx, float* inv_den, float* scale,
    int64_t B, int64_t H, int64_t W, int64_t C, void* workspace, size_t workspace_bytes,
    void* stream);

/* 1x1 convolution on channels-last bf16 maps as a GEMM on the matrix cores:
 * out [M, N] = epi(x' [M, K] . weight^T + bias) with weight [N, K] bf16 (the 1x1
 * kernel as stored, cast to bf16 as autocast casts it), bias [N] fp32 (or NULL),
 * M = B*H*W pixels, K % 32 == 0, N % 32 == 0,
 * 16-byte aligned tensors.  The linear result is rounded to bf16 first, as the
 * reference's autocast linear output is; then
 *   epilogue 0: out = that value                              (proj_in, local_gate, W_q, proj_out)
 *   epilogue 1: out = bf16(gelu(that value))                  (ffn.fc1 + ffn.act)
 *   epilogue 2: out = bf16(residual + that value), residual [M, N] bf16  (ffn.fc2 + residual add)
 *   epilogue 3: out = bf16(silu(that value))                  (head_pre_logits + folded head_norm + head_act)
 * With grn_scale [M / pixels_per_image, K] and grn_beta [K] (both fp32, or both NULL)
 * the operand is x' = bf16(x * grn_scale[image] + grn_beta), the GRN output the
 * reference feeds to ffn.fc2 (vh_grn_scale_forward gives the scale).  No counterpart
 * in the reference's native code: it runs nn.Conv2d / nn.Linear and the GELU, GRN,
 * residual add and SiLU as separate ops (models/block.py:70-107, models/layers.py:67-80,
 * models/hierarchical.py:62-84). */
int vh_pointwise_conv_nhwc_forward(
    const void* x, int32_t io_dtype, const void* weight, const float* bias, int32_t epilogue,
    const void* residual, const float* grn_scale, const float* grn_beta, int64_t pixels_per_image,
    void* out, int64_t M, int64_t N, int64_t K, void* stream);

/* Two chained 1x1 convolutions of the same pixels, as two vh_pointwise_conv_nhwc_forward
 * calls with the bias epilogue give them: out [M, N] = bf16(x @ weight^T + bias) and out2
 * [M, N] = bf16(out @ weight2^T + bias2), bf16 operands (x [M, K], weight [N, K], weight2
 * [N, N]), FP32 biases or NULL, N = 64 or 128 with K % 64 == 0, or N = 32 with K = 32 or 64,
 * 16-byte aligned.  One launch:
 * each block keeps its rows of out in LDS for the second product.  No counterpart in the
 * reference (its block runs proj_in, then local_gate on the result: models/block.py:63-66). */
int vh_pointwise_chain_nhwc_forward(
    const void* x, const void* weight, const float* bias, const void* weight2, const float* bias2,
    void* out, void* out2, int64_t M, int64_t N, int64_t K, void* stream);

/* A 1x1 convolution with the residual add and the LayerNorm that follow it in the block
 * (proj_out, then norm2 of the sum), in one launch: out_sum [M, N] = bf16(residual +
 * bf16(x @ weight^T + bias)) and out_norm [M, N] = bf16(LayerNorm(out_sum)) over the N
 * channels of each pixel (ln_weight, ln_bias [N] fp32, eps), all bf16 but the affine and
 * bias; N = 64 with K = 32 or 64, or N = 128 or 256 with K = 64 or 128; 16-byte aligned.
 * The bits of vh_pointwise_conv_nhwc_forward (bias epilogue) followed by
 * vh_add_layernorm2d_forward: the LayerNorm sums run in that kernel's order.  No
 * counterpart in the reference (its block adds the branch and applies norm2 in separate
 * steps: models/block.py:104-106). */
int vh_pointwise_add_layernorm_nhwc_forward(
    const void* x, const void* weight, const float* bias, const void* residual, const float* ln_weight,
    const float* ln_bias, float eps, void* out_sum, void* out_norm, int64_t M, int64_t N, int64_t K, void* stream);

/* 3x3 convolution, padding 1, stride 1 or 2, on a channels-last map as an implicit GEMM
 * on the matrix cores: out [B, Ho, Wo, N] bf16 = act(bf16(conv(x, weight) + bias)),
 * rounded to bf16 after the sum and after the activation (act 0 = none, 1 = exact GELU).
 * x [B, H, W, Cin] bf16 with Cin % 32 == 0, or Cin = 3 (the image: fp32, rounded to
 * bf16 on load as autocast rounds it, or bf16).  weight bf16 [N, K]: for Cin % 32 == 0
 * the convolution weight in channels-last order [N, 3, 3, Cin] (K = 9 Cin); for Cin = 3,
 * K = 64 with weight[n][4 (3 kh + kw) + c] and zeros at c = 3 and taps 9..15.  bias [N]
 * fp32.  N a multiple of 32; Ho = (H - 1) / stride + 1, likewise Wo;
 * weight, bias, out (and x unless Cin = 3) 16-byte aligned.  With an eval-mode
 * BatchNorm folded into weight and bias this is Conv2d + BatchNorm2d (+ GELU) of the
 * stem and the downsample layers (models/layers.py:85-119).  No counterpart in the
 * reference's native code (it runs nn.Conv2d, nn.BatchNorm2d and nn.GELU). */
int vh_conv3x3_nhwc_forward(
    const void* x, int32_t x_dtype, const void* weight, const float* bias, int32_t act, void* out,
    int64_t batch, int64_t height, int64_t width, int64_t in_channels, int64_t out_channels,
    int32_t stride, void* stream);

/* Per-channel bias and optional exact GELU on a channels-last map x [pixels, C]
 * (io_dtype, C % 8 == 0, 16-byte aligned; out may alias x):
 * out = act(round(x + bias)), act 0 = identity, 1 = GELU, rounded to io_dtype after
 * each step.  With a BatchNorm folded into the preceding convolution's weights this
 * is the BatchNorm output and its activation in the stem and downsample layers
 * (models/layers.py:85-119).  No counterpart in the reference's native code (it runs
 * nn.BatchNorm2d and nn.GELU). */
int vh_bias_act_nhwc_forward(
    const void* x, int32_t io_dtype, const float* bias, int32_t act, void* out,
    int64_t total, int64_t channels, void* stream);

/* Residual add on channels-last data: out[i] = residual[i] +
 * branch[i] * gamma[c] * drop_scale[b] (fp32 out; residual/branch io_dtype
 * each).  Replaces the Triton _residual_forward_kernel (utils/residual.py:31-52). */
int vh_residual_add_forward(
    const void* residual, int32_t residual_dtype, const void* branch, int32_t branch_dtype,
    const float* gamma, const float* drop_scale, float* out,
    int64_t total, int64_t channels, int64_t spatial, void* stream);

/* Direction fusion backward (replaces visionhope_postprocess_scale_backward,
 * utils/csrc/direction_fusion.cpp:2, direction_fusion.cu:123-691, bound at
 * utils/direction_fusion.py:108-120).  dout: FP32 [B, C, H, W] (channels-last storage if
 * dout_channels_last, else NCHW); y, x: [B, 4, heads, H*W, head_dim] in io_dtype; dy, dx:
 * same layout and dtype; d_dskip: FP32 [C] or [4, C] (skip_per_dir); d_scale: FP32 [4, C].
 * Parameter gradients are summed in a fixed order (deterministic). */
size_t vh_postprocess_scale_backward_workspace_bytes(int64_t B, int64_t heads, int64_t H, int64_t W,
                                                     int32_t head_dim, int32_t skip_per_dir);
int vh_postprocess_scale_backward(const float* dout, int32_t dout_channels_last, const void* y, const void* x,
                                  int32_t io_dtype, const float* d_skip, int32_t skip_per_dir, const float* scale,
                                  void* dy, void* dx, float* d_dskip, float* d_scale, int64_t B, int64_t heads,
                                  int64_t H, int64_t W, int32_t head_dim, void* workspace, size_t workspace_bytes,
                                  void* stream);

/* GRN backward (replaces grn_backward_cuda, utils/csrc/grn.cpp:4-11, grn_cuda.cu:126-359,
 * bound at utils/grn_cuda.py:51-82).  dout: FP32 channels-last [B, C, H, W]; x: the forward
 * input (channels-last, io_dtype); gx [B, C] and inv_den [B] as written by vh_grn_forward;
 * dx: channels-last in io_dtype; dgamma, dbeta: FP32 [C]. */
size_t vh_grn_backward_workspace_bytes(int64_t B, int64_t C, int64_t H, int64_t W);
int vh_grn_backward(const float* dout, const void* x, int32_t io_dtype, const float* gamma, const float* gx,
                    const float* inv_den, void* dx, float* dgamma, float* dbeta, int64_t B, int64_t C, int64_t H,
                    int64_t W, void* workspace, size_t workspace_bytes, void* stream);

/* LayerNorm2d backward (replaces the Triton _layernorm2d_backward_kernel and
 * _layernorm2d_reduce_kernel, utils/layer_norm_cuda.py:59-121,148-192).  dy: FP32
 * channels-last; x: the forward input (channels-last, io_dtype); mean, rstd: [B*H*W] as
 * written by vh_layernorm2d_forward; dx: channels-last in io_dtype; dweight, dbias: FP32
 * [C].  C <= 1024. */
size_t vh_layernorm2d_backward_workspace_bytes(int64_t B, int64_t C, int64_t H, int64_t W);
int vh_layernorm2d_backward(const float* dy, const void* x, int32_t io_dtype, const float* weight, const float* mean,
                            const float* rstd, void* dx, float* dweight, float* dbias, int64_t B, int64_t C,
                            int64_t H, int64_t W, void* workspace, size_t workspace_bytes, void* stream);

/* Query normalisation backward (replaces visionhope_qnorm_backward,
 * utils/csrc/query_normalization.cpp:3, query_normalization.cu:78-134).  dq_out, q_out:
 * FP32 [B, R, heads, N, d]; inv_norm: [B, R, heads, N] as written by vh_qnorm_forward;
 * dq_raw: [B, R, N, heads*d] in io_dtype. */
int vh_qnorm_backward(const float* dq_out, const float* q_out, const float* inv_norm, void* dq_raw, int32_t io_dtype,
                      int64_t B, int64_t R, int64_t N, int64_t heads, int32_t head_dim, void* stream);

/* Residual add backward (replaces the Triton _residual_backward_kernel and
 * _residual_reduce_kernel, utils/residual.py:55-101,132-170).  dout: FP32 channels-last
 * [B, C, H, W] (total = B*C*H*W values, spatial = H*W); branch: the forward's branch in
 * branch_dtype; gamma [C], mask [B] FP32; dbranch in branch_dtype; dgamma FP32 [C].
 * The residual's gradient is dout itself. */
size_t vh_residual_add_backward_workspace_bytes(int64_t total, int64_t channels);
int vh_residual_add_backward(const float* dout, const void* branch, int32_t branch_dtype, const float* gamma,
                             const float* mask, void* dbranch, float* dgamma, int64_t total, int64_t channels,
                             int64_t spatial, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VISIONHOPE_HIP_H */
