/*
 * wohper_hip.h - C ABI of the MI355X (gfx950) decode hot path.
 *
 * Drop-in boundary for the reference engine's DeepSeek-V4 kernel entry points
 * (Twenytwo/wohper, engine/zc_infer_core/src = E/).  Every hot-path function
 * below names the reference function it replaces.  The reference is Rust; its
 * binding is an `extern "C"` block behind a `rocm` cargo feature (see
 * INTEGRATION.md).  Plain pointers and sizes only.
 *
 * Ownership: the caller owns every host buffer; the library never frees
 * caller memory.  Device weights are owned by the context's weight store for
 * the context's lifetime (or until wh_store_release).  All functions are
 * thread-compatible: one context (one HIP stream) per engine thread.
 *
 * Synchronous entry points take host slices and return after the result is
 * in the caller's buffer (the reference's semantics).  *_async entry points
 * take device pointers, are ordered on the context stream, and report
 * failures through wh_stream_status().
 */
#ifndef WOHPER_HIP_H
#define WOHPER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  1..8 mirror DeepSeekV4KernelError (E/deepseek_v4.rs:398-408)
 * in order; the rest cover ComputeError cases of the FP8 path
 * (E/compute.rs:6180-6215), the weight store and the HIP runtime. */
enum wh_status {
    WH_OK = 0,
    WH_EMPTY_SHAPE = 1,
    WH_INVALID_SHAPE = 2,
    WH_PACKED_WEIGHT_TOO_SMALL = 3,
    WH_SCALE_TOO_SMALL = 4,
    WH_INPUT_TOO_SMALL = 5,
    WH_OUTPUT_TOO_SMALL = 6,
    WH_SCRATCH_TOO_SMALL = 7,
    WH_NON_FINITE_OUTPUT = 8,
    WH_INVALID_QUANT_FORMAT = 9,   /* e.g. "DeepSeek FP8 scale is not UE8M0" */
    WH_NOT_RESIDENT = 10,          /* unknown tensor handle or (layer, expert) key */
    WH_OUT_OF_MEMORY = 11,
    WH_HIP_ERROR = 12,
    WH_INVALID_ARGUMENT = 13,
    WH_NON_FINITE_INPUT = 14,      /* reserved: inputs with inf/NaN follow the reference's
                                      act-quant (NaN -> -480 x scale; an inf makes the
                                      block scale inf and surfaces as NonFiniteOutput) */
    WH_UNSUPPORTED = 15,
    /* ZCBLK01 block errors: ComputeError (E/compute.rs:330-344); the
     * reference's Display text of the error is in wh_last_error() */
    WH_TRUNCATED_QUANT_BLOCK = 16,           /* TruncatedQuantBlock(field) */
    WH_INVALID_QUANT_BLOCK_MAGIC = 17,       /* InvalidQuantBlockMagic */
    WH_UNSUPPORTED_QUANT_BLOCK_VERSION = 18, /* UnsupportedQuantBlockVersion */
    WH_INVALID_QUANT_BLOCK = 19,             /* InvalidQuantBlock(reason) */
    WH_TENSOR_INDEX_OUT_OF_RANGE = 20,       /* TensorIndexOutOfRange */
    /* experts-pack errors: ModelFormatError (E/model_format.rs:32-56) */
    WH_UNALIGNED = 21,                       /* Unaligned{field, value} */
    WH_IO_ERROR = 22                         /* Io: open/read of the pack file */
};

/* Scale formats of an FP8 block-scaled tensor. */
enum wh_scale_format {
    WH_SCALE_UE8M0 = 0, /* one byte per block: 2^(b-127), 0 -> 0.0, 255 -> inf */
    WH_SCALE_F32 = 1    /* one float per block */
};

typedef struct wh_ctx wh_ctx;
typedef uint64_t wh_tensor; /* handle into the weight store, 0 = none */

/* One routed expert of a token: IoBlockPtr{layer_id, expert_id, route_weight}
 * (E/compute.rs:896-904) without the host pointer - experts are resident. */
typedef struct {
    uint32_t layer_id;
    uint32_t expert_id;
    float route_weight;
} wh_expert_route;

/* ----------------------------------------------------------- lifecycle */
int wh_init(int device, wh_ctx** out);
int wh_shutdown(wh_ctx* ctx);
const char* wh_status_string(int status);
/* Blocks until the stream drains; returns the first deferred kernel status
 * (WH_NON_FINITE_OUTPUT, WH_NOT_RESIDENT) raised since the last call. */
int wh_synchronize(wh_ctx* ctx);
/* The context's hipStream_t, for callers that interleave their own work. */
void* wh_stream(wh_ctx* ctx);
/* Text of the last HIP runtime failure on this thread (empty if none). */
const char* wh_last_error(void);
/* Library build description (architecture, libm table sizes). */
const char* wh_build_info(void);

/* --------------------------------------------------------- weight store
 * Replaces the SSD/page-cache streaming path of the reference
 * (E/direct_io.rs:575-681, E/scheduler.rs:148-194, E/server/generation.rs:196-306):
 * tensors are re-laid out once for the GPU kernels and stay in HBM. */

/* FP8 E4M3 weight [rows x cols] with block scales [scale_rows x scale_cols]
 * (E/compute.rs:6174-6215 shape rules: rows % scale_rows == cols % scale_cols == 0). */
int wh_store_fp8(wh_ctx* ctx, const uint8_t* weight, size_t weight_len, size_t rows, size_t cols,
                 const void* scales, size_t scales_len, int scale_format, size_t scale_rows,
                 size_t scale_cols, wh_tensor* out);

/* FP4 E2M1 packed weight [rows x ceil(cols/2)] (low nibble = even column) with
 * UE8M0 scales [rows x scale_cols]: the Fp4Matvec of E/deepseek_v4.rs:410-417,
 * validated as validate_fp4_matvec (E/deepseek_v4.rs:434-462). */
int wh_store_fp4(wh_ctx* ctx, const uint8_t* packed, size_t packed_len, const uint8_t* scales,
                 size_t scales_len, size_t rows, size_t cols, size_t scale_cols, wh_tensor* out);

/* Registers an FP4 SwiGLU expert (DeepSeekV4Fp4Expert, E/deepseek_v4.rs:419-424)
 * under the (layer_id, expert_id) key the engine routes by.  Shapes are checked
 * as in deepseek_v4_fp4_expert_from_quant_block (E/compute.rs:1249-1268). */
int wh_store_expert(wh_ctx* ctx, uint32_t layer_id, uint32_t expert_id, wh_tensor w1, wh_tensor w3,
                    wh_tensor w2);

/* ------------------------------------------------------ ZCBLK01 blocks
 * The engine's expert blocks as they come off disk (one ZCBLK01 block per
 * (layer, expert), E/direct_io.rs ReadTicket -> IoBlockPtr{ptr, len}).
 * Parsing follows parse_quant_block (E/compute.rs:1099-1148) and
 * QuantBlockLayout::tensor (E/compute.rs:545-600) check for check; a bad
 * block returns the status of the reference's error and wh_last_error()
 * holds its Display text (e.g. "truncated ZCBLK field: record table").
 * The three functions below read only host memory and need no device. */

/* One tensor record (QuantTensorLayout, E/compute.rs:441-451) resolved
 * against the block: offsets are absolute byte offsets into the block. */
typedef struct {
    uint16_t dtype_original;
    uint16_t quant_format;  /* 2401 FP8 E4M3, 2402 FP4 E2M1 packed, 2403 UE8M0 */
    uint32_t rank;
    uint32_t flags;         /* TensorRole code in the low 16 bits */
    float scale;
    float zero_point;
    size_t name_offset;     /* name bytes (no terminator) */
    size_t name_len;
    size_t shape_offset;    /* {u32 rank, rank x u64 dims} */
    size_t data_offset;
    size_t data_bytes;
} wh_quant_tensor;

/* One FP4 projection of an expert block (Fp4Matvec, E/deepseek_v4.rs:411-417):
 * packed weight [rows x cols/2] and UE8M0 scales [rows x scale_cols] as byte
 * ranges of the block. */
typedef struct {
    size_t rows, cols, scale_cols;
    size_t weight_offset, weight_bytes;
    size_t scale_offset, scale_bytes;
} wh_fp4_view;

/* parse_quant_block (E/compute.rs:1099-1148): header fields of a block. */
int wh_quant_block_header(const uint8_t* block, size_t block_len, uint32_t* tensor_count,
                          uint32_t* quant_format, uint32_t* flags);
/* parse_quant_block + QuantBlockLayout::tensor(index) (E/compute.rs:545-600). */
int wh_quant_block_tensor(const uint8_t* block, size_t block_len, size_t index, wh_quant_tensor* out);
/* deepseek_v4_fp4_expert_from_quant_block (E/compute.rs:1249-1268): the
 * w1 (gate), w3 (up), w2 (down) projections found by name suffix. */
int wh_quant_block_fp4_expert(const uint8_t* block, size_t block_len, wh_fp4_view out[3]);

/* Makes the FP4 expert of a ZCBLK01 block resident under (layer_id,
 * expert_id).  Replaces the per-decode parse of the block the IO scheduler
 * delivered (compute_expert_block -> deepseek_v4_fp4_expert_from_quant_block,
 * E/compute.rs:5467-5478, 5636): the block is parsed and uploaded once.
 * An expert already stored under the key is replaced. */
int wh_store_expert_block(wh_ctx* ctx, uint32_t layer_id, uint32_t expert_id, const uint8_t* block,
                          size_t block_len);

/* One entry of the experts-pack index <model>.experts_pack.index.json
 * (ExpertPackEntryDisk, E/model_format.rs:448-455). */
typedef struct {
    uint32_t layer_id;
    uint32_t expert_id;
    uint64_t offset;        /* 2 MB aligned */
    uint64_t disk_bytes;    /* 2 MB aligned */
    uint64_t payload_bytes; /* the ZCBLK01 block: the first payload_bytes at offset */
} wh_expert_pack_entry;

/* Loads the listed experts of a consolidated experts pack into the store:
 * the reads the reference's scheduler queues per decode step
 * (E/scheduler.rs:163-176, fixed file #1) done once, each block parsed as by
 * wh_store_expert_block.  Entries are checked as load_optional_expert_pack
 * does (E/model_format.rs:488-491: offset and disk_bytes 2 MB aligned) before
 * any read; payload_bytes > disk_bytes is rejected too.  Reads of the next
 * block overlap the upload of the previous one.  *stored counts the experts
 * made resident (all of them on WH_OK; the ones before the failing entry
 * otherwise). */
int wh_store_expert_pack(wh_ctx* ctx, const char* pack_path, const wh_expert_pack_entry* entries, size_t n,
                         size_t* stored);

/* ---------------------------------------------------------------- router
 * route_experts_from_dense_block (E/compute.rs:2129-2268) on the GPU: the
 * gate GEMV (bf16 in the x86 lane order of dot_bf16_row_avx2,
 * E/compute.rs:6116-6136, or the FP8 GEMV), sqrt-softplus, the biased top-k
 * or the hash layer's tid2eid row, and finalize_route_weights - bit-exact,
 * so the routed experts can follow without a host round trip. */

/* RouterMath (E/compute.rs:408-417) */
enum wh_router_math {
    WH_ROUTER_RAW_LOGITS = 0,     /* raw gate outputs, no bias, no normalisation */
    WH_ROUTER_SQRT_SOFTPLUS = 1   /* DeepSeekV4SqrtSoftplus */
};

/* RouteOptions (E/compute.rs:2096-2127). hash_token_id < 0: none. */
typedef struct {
    int32_t math;
    float route_scale;
    int64_t hash_token_id;
} wh_route_options;

/* Makes the router of a layer's dense ZCBLK01 block resident: the gate
 * (router_gate_tensor, E/compute.rs:2444-2467: the Router-role matrix whose
 * cols equal hidden_len, else the first; bf16 or FP8 with its UE8M0 scale),
 * the selection bias (router_bias_values, E/compute.rs:2335-2376) and the
 * tid2eid table (router_tid2eid_tensor, E/compute.rs:2270-2285).  *found = 0
 * when the block has no gate (the reference's Ok(None)); a router already
 * stored for the layer is replaced.  Up to 1024 experts. */
int wh_store_router(wh_ctx* ctx, uint32_t layer_id, const uint8_t* block, size_t block_len, size_t hidden_len,
                    int* found);

/* route_experts_from_dense_block on host slices: hidden [hidden_len] in,
 * the selected experts' ids and weights out (*n_out <= active_experts).
 * available = NULL means every gate row, in id order; ids past the gate's
 * rows have no score and are dropped.  active_experts <= 64,
 * n_available <= 1024.  WH_NOT_RESIDENT when the layer has no router. */
int wh_route_experts(wh_ctx* ctx, uint32_t layer_id, const float* hidden, size_t hidden_len, size_t active_experts,
                     const uint32_t* available, size_t n_available, const wh_route_options* options,
                     uint32_t* expert_ids, float* scores, size_t out_cap, size_t* n_out);

/* The same on device pointers, ordered on the context stream: x_dev
 * [hidden_len] f32 (16-byte aligned), available_dev (or NULL), outputs ids_dev / scores_dev
 * [active_experts] and count_dev.  Argument and table errors are returned
 * here, before anything is queued. */
int wh_route_experts_async(wh_ctx* ctx, uint32_t layer_id, const float* x_dev, size_t hidden_len,
                           size_t active_experts, const uint32_t* available_dev, size_t n_available,
                           const wh_route_options* options, uint32_t* ids_dev, float* scores_dev,
                           uint32_t* count_dev);

/* Device-side synthetic fill of an FP4 expert with the counter-based RNG of
 * the benchmark (uniform packed bytes, UE8M0 bytes in [scale_lo, scale_hi]),
 * written directly in the resident layout - for stacks too large to stage
 * through the host.  Identical bytes to wh_synth_fp4_host. */
int wh_store_expert_synthetic(wh_ctx* ctx, uint32_t layer_id, uint32_t expert_id, size_t hidden,
                              size_t inter, uint64_t seed, uint32_t scale_lo, uint32_t scale_hi);

/* Synthetic FP8 tensor generated on the device straight into the resident
 * layout (no host copy of the bytes), for stacks too large to upload: byte i
 * of the row-major original is wh_synth_fp8_host's byte i, approximately
 * uniform over the 254 finite E4M3 codes.  Scales are f32, 128x128 blocks.
 * No counterpart in the reference (its weights come from checkpoints). */
int wh_store_fp8_synthetic(wh_ctx* ctx, size_t rows, size_t cols, uint64_t seed, uint64_t stream,
                           const float* scales, size_t scale_rows, size_t scale_cols, wh_tensor* out);
void wh_synth_fp8_host(uint64_t seed, uint64_t stream, uint8_t* weight, size_t n);

/* Host generator of the same bytes (original reference layout). */
void wh_synth_fp4_host(uint64_t seed, uint64_t stream, uint8_t* packed, size_t packed_len,
                       uint8_t* scales, size_t scales_len, uint32_t scale_lo, uint32_t scale_hi);

int wh_store_release(wh_ctx* ctx, wh_tensor t);
int wh_store_usage(wh_ctx* ctx, size_t* device_bytes, size_t* tensors, size_t* experts);

/* Bit-exact dequantisation of a resident tensor back to reference values, in
 * the original column order: FP4 -> decode_fp4_e2m1(nibble, scale)
 * (E/deepseek_v4.rs:358-372); FP8 -> decode_fp8_e4m3(byte, 1.0)
 * (E/deepseek_v4.rs:151-164, scales not applied).  out: rows*cols floats. */
int wh_tensor_dequant(wh_ctx* ctx, wh_tensor t, float* out, size_t out_len);

/* ------------------------------------------------------------- hot path */

/* gemv_fp8_e4m3_ue8m0_tensorwise (E/compute.rs:6174) when row_start == 0 and
 * row_end == rows, else gemv_fp8_e4m3_ue8m0_rows (E/compute.rs:6244): output
 * gets row_end - row_start values; *values_out = weight values consumed, as
 * the reference's Ok(usize). */
int wh_fp8_gemv(wh_ctx* ctx, wh_tensor w, size_t row_start, size_t row_end, const float* input,
                size_t input_len, float* output, size_t output_len, size_t* values_out);

/* gemv_fp8_e4m3_ue8m0_rows_multi (E/compute.rs:6384): n inputs of length
 * cols at stride input_stride, n outputs at stride output_stride. */
int wh_fp8_gemv_multi(wh_ctx* ctx, wh_tensor w, size_t row_start, size_t row_end,
                      const float* inputs, size_t n, size_t input_stride, float* outputs,
                      size_t output_stride, size_t* values_out);

/* fp4_e2m1_ue8m0_matvec_scalar (E/deepseek_v4.rs:464). */
int wh_fp4_matvec(wh_ctx* ctx, wh_tensor w, const float* input, size_t input_len, float* output,
                  size_t output_len);

/* deepseek_v4_fp4_expert_forward_scalar (E/deepseek_v4.rs:561): scratch_len is
 * the caller's scratch size in floats (checked like the reference, >= 2*inter;
 * the device keeps its own scratch). */
int wh_fp4_expert_forward(wh_ctx* ctx, uint32_t layer_id, uint32_t expert_id, const float* input,
                          size_t input_len, float* output, size_t output_len, size_t scratch_len);

/* fp8_act_quant_dequant_in_place (E/compute.rs:2504). */
int wh_act_quant_dequant(wh_ctx* ctx, float* values, size_t n, size_t block_size);

/* compute_active_experts (E/compute.rs:1948): hidden (len >= hidden size) is
 * replaced by the route-weighted sum of the experts' outputs, in route order. */
int wh_routed_experts(wh_ctx* ctx, const wh_expert_route* routes, size_t n_routes, float* hidden,
                      size_t hidden_len);

/* Routed experts plus the shared expert, replacing
 * compute_active_and_shared_experts (E/compute.rs:1872-1946): hidden =
 * shared(x), then hidden += the routed sum of wh_routed_experts.  The shared
 * expert is a resident expert keyed (shared_layer, shared_expert); n may be 0
 * (shared expert only).  The async variant takes device pointers like
 * wh_routed_experts_async. */
int wh_routed_and_shared_experts(wh_ctx* ctx, const wh_expert_route* routes, size_t n_routes,
                                 uint32_t shared_layer, uint32_t shared_expert, float* hidden,
                                 size_t hidden_len);
int wh_routed_and_shared_experts_async(wh_ctx* ctx, const wh_expert_route* routes, size_t n_routes,
                                       uint32_t shared_layer, uint32_t shared_expert, const void* x_dev,
                                       int x_is_bf16, size_t n_tokens, float* out_dev);

/* wh_routed_and_shared_experts_async for one token whose route list is in
 * device memory, as wh_route_experts_async leaves it: count_dev[0] routes
 * (at most n_slots are taken; n_slots >= 1 and at most 15 with a shared
 * expert, 16 without)
 * of layer_id, expert ids_dev[i] with weight weights_dev[i], in route order.
 * The list is resolved against the layer's resident experts on the device,
 * so a router on the device feeds the experts with no host round trip: the
 * reference routes a decode token (route_experts_from_dense_block,
 * E/compute.rs:2129-2268) and then runs compute_active_and_shared_experts
 * (E/compute.rs:1872-1946) on those routes.  Every resident expert of the
 * layer and the shared expert (WH_NO_SHARED_EXPERT: none) must share one
 * shape the fast kernels take (else WH_UNSUPPORTED).  An id with no resident
 * expert reports WH_NOT_RESIDENT through wh_stream_status. */
int wh_routed_and_shared_experts_dev_async(wh_ctx* ctx, uint32_t layer_id, const uint32_t* ids_dev,
                                           const float* weights_dev, const uint32_t* count_dev, size_t n_slots,
                                           uint32_t shared_layer, uint32_t shared_expert, const void* x_dev,
                                           int x_is_bf16, float* out_dev);

/* Allocation-free variant of wh_routed_and_shared_experts_async, same
 * arguments and results.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  It calls no allocating
 * routine; its working memory (SwiGLU outputs, per-expert outputs, routed-sum
 * arrival counters) is one fixed array of
 * WH_NOALLOC_SCRATCH_BYTES per GPU, set up by wh_init and held until the
 * process ends.  Every call on a GPU shares that GPU's array, so calls that
 * overlap on one GPU (other contexts, other threads' streams) race; calls on
 * one context's stream are ordered.  Only experts on the fast kernels'
 * shapes are taken (else WH_UNSUPPORTED); a call whose working memory,
 * about n_tokens x (n_routes + 1) x 4 x (hidden + intermediate) bytes,
 * exceeds the array returns WH_SCRATCH_TOO_SMALL before anything is
 * queued, with the sizes in wh_last_error(). */
#define WH_NOALLOC_SCRATCH_BYTES (8u << 20)
int wh_routed_and_shared_experts_noalloc_async(wh_ctx* ctx, const wh_expert_route* routes, size_t n_routes,
                                               uint32_t shared_layer, uint32_t shared_expert, const void* x_dev,
                                               int x_is_bf16, size_t n_tokens, float* out_dev);

/* compute_deepseek_fp8_shared_expert_into_hidden (E/compute.rs:5545-5614):
 * output[..w2 rows] = W2 act_quant(swiglu(W1 xq, W3 xq)) with
 * xq = act_quant(input) (block 64), each stage bit-identical to the
 * reference.  w1/w3/w2 are resident FP8 tensors (wh_store_fp8); shapes are
 * checked as the reference does ("DeepSeek shared expert input dim",
 * "... projection shape" -> WH_INVALID_SHAPE; w2 rows beyond output_len ->
 * WH_OUTPUT_TOO_SMALL).  The async variant takes device pointers (f32; x and
 * y may alias, like the reference's in-place hidden_states). */
int wh_fp8_shared_expert(wh_ctx* ctx, wh_tensor w1, wh_tensor w3, wh_tensor w2, const float* input,
                         size_t input_len, float* output, size_t output_len);
int wh_fp8_shared_expert_async(wh_ctx* ctx, wh_tensor w1, wh_tensor w3, wh_tensor w2, const float* x_dev,
                               float* y_dev);

/* Numerics of the routed/shared expert entry points above, of
 * wh_fp4_expert_forward and of the batch entry points below.  on = 1 (the
 * default): every matvec follows the
 * reference CPU kernel's summation order (E/deepseek_v4.rs:294-347), so
 * outputs are bit-identical to it.  on = 0: for the model's expert shapes
 * (hidden 2048 or 4096, inter 2048) block-scaled FP8 MFMA kernels take the
 * reference's exact operands (E4M3 codes of the act-quantized inputs and of
 * the FP4 LUT values, UE8M0 / E8M0 block scales) and free only the summation
 * order; the dequantized weights are the reference's values exactly and each
 * matvec agrees with the reference kernel on the same input within
 * max|diff| <= 1e-5 * ||w_row||_2 * ||x||_2 (fp32 accumulation), while
 * act-quant, SwiGLU and the route-weighted sum stay bit-exact given the
 * matvec outputs.  on = 0 also frees the order of the FP8 dequant GEMV
 * (wh_fp8_gemv*, the shared expert, the multi-input GEMV below its MFMA
 * threshold) on tensors of a multiple of 1024 columns whose codes avoid
 * 0x7F / 0xFF, to the same bound; the router's FP8 gate keeps the reference
 * order in both modes (its top-k selection must not move).  No counterpart
 * in the reference (it has one CPU kernel). */
int wh_set_exact_numerics(wh_ctx* ctx, int on);
/* Test support, no counterpart in the reference: with capture on, the
 * routed-expert entry points also keep each expert's gate and up matvec
 * outputs; wh_debug_moe_token_read copies a buffer of the last call (T
 * tokens, n experts including the shared one) to host.  which: 0 gate/up
 * (f32 [T][n][2][inter], gate then up; capture must be on), 1 SwiGLU
 * outputs (f32 [T][n][inter]), 2 expert outputs (f32 [T][n][hidden]). */
int wh_debug_moe_token_capture(wh_ctx* ctx, int on);
int wh_debug_moe_token_read(wh_ctx* ctx, int which, void* out, size_t bytes);
/* Measurement support, no counterpart in the reference: which kernels the
 * MFMA numerics mode runs for a token at hidden 4096, inter 2048 and up to
 * 8 experts.  mask bit 0: gate/up, bit 1: down streamed into LDS by direct
 * loads; a clear bit: the register-ring kernel of that stage (also used for
 * every other shape).  The default, 1, is the faster pair measured in the
 * token pipeline.  All compute the same operands; only the fp32 summation
 * order differs. */
int wh_debug_token_kernels(wh_ctx* ctx, int mask);

/* Batched routed experts for npos positions, expert-major, replacing the
 * batch-prefill MoE of the reference: per-position weights score / sum (or
 * 1 / topk when the sum is not finite and positive or a score is not finite)
 * and the union of selected experts (E/server/generation.rs:2487-2506), then
 * for each expert in ascending id and each of its positions
 * acc_p += y * w, unfused, from 0 (accumulate_expert_for_positions,
 * E/compute.rs:1779-1810).  With a shared expert (shared_expert !=
 * WH_NO_SHARED_EXPERT), out_p = shared(x_p) + acc_p
 * (finish_layer_deepseek_mhc_phase2_batch, E/compute.rs:1838-1852).
 * route_ids / route_scores: [npos][topk] expert ids of layer_id and their
 * router scores.  x: [npos][hidden]; out: [npos][hidden].  The reference
 * takes expert blocks in I/O completion order; this takes them in ascending
 * id, its submission order.  A route id that is not resident returns
 * WH_NOT_RESIDENT (the async variant reports it through the stream status).
 * The async variant takes device pointers (x f32 or bf16) and enqueues on
 * the library stream; the grouping runs on the device. */
/* With exact numerics off (wh_set_exact_numerics(ctx, 0)), experts of a
 * batch with at least min_tokens tokens run on block-scaled FP8 MFMA (E4M3
 * codes of the weights' x8 LUT values and of the act-quantized inputs, E8M0
 * block scales, fp32 accumulation): their outputs agree with the reference
 * within fp32 rounding of a different summation order; the other experts
 * stay bit-identical to the reference's AVX2 kernel.  Default 1 (every
 * expert: the MFMA items stream the weights faster than the exact ones even
 * for one token); 0 keeps every expert on the exact path, as exact numerics
 * do whatever the threshold.  No counterpart in the reference (its batch
 * path has one kernel). */
int wh_set_moe_mfma_min(wh_ctx* ctx, uint32_t min_tokens);
/* Test support for the batch path, no counterpart in the reference:
 * copies a device buffer of the last single-chunk fast batch call (S = its
 * slots) to host.  which: 0 assignment of each slot (u32 [S]), 1 gate
 * matvecs (f32 [S][inter]), 2 up matvecs (f32 [S][inter]), 3 expert outputs
 * (f32 [S][hidden]), 4 meta (u32 [8]: used experts, routes valid, queues,
 * experts on MFMA), 5 slot ranges of the used experts (u32 [S + 1]), 6 used
 * expert ids (u32 [S]), 7 work order (u32 [S]), 8 act-quantized SwiGLU
 * outputs (f32 [S][inter]). */
int wh_debug_moe_batch_read(wh_ctx* ctx, int which, void* out, size_t bytes);
#define WH_NO_SHARED_EXPERT 0xFFFFFFFFu
int wh_moe_batch(wh_ctx* ctx, uint32_t layer_id, const uint32_t* route_ids, const float* route_scores, size_t npos,
                 size_t topk, uint32_t shared_layer, uint32_t shared_expert, const float* x, size_t x_len,
                 float* out, size_t out_len);
int wh_moe_batch_async(wh_ctx* ctx, uint32_t layer_id, const uint32_t* route_ids_dev,
                       const float* route_scores_dev, size_t npos, size_t topk, uint32_t shared_layer,
                       uint32_t shared_expert, const void* x_dev, int x_is_bf16, float* out_dev);

/* Device-pointer variant for the resident decode path: x_dev holds n_tokens
 * rows of `hidden` values (f32, or bf16 when x_is_bf16), all routed to the same
 * expert list; out_dev gets n_tokens rows of f32.  Stream-ordered. */
int wh_routed_experts_async(wh_ctx* ctx, const wh_expert_route* routes, size_t n_routes,
                            const void* x_dev, int x_is_bf16, size_t n_tokens, float* out_dev);

/* Several device-pointer FP8 GEMVs enqueued by one call, in order (a decode
 * layer's projections: the reference calls gemv_fp8_e4m3_ue8m0_rows once per
 * projection and per wo_a group, E/compute.rs:4005-4265).  Every descriptor
 * is validated before the first launch.  A run of consecutive descriptors on
 * one tensor with equal, adjacent row groups (a power of two of at least 8
 * rows), evenly spaced inputs and back-to-back outputs goes out as one
 * launch; so do two consecutive descriptors of different tensors on the same
 * input (wq_a and wkv) when the tensors share width, scale format and the
 * special-code flag and neither output overlaps the input or the other
 * output.  Any other descriptor is a launch of its own.  Results are the
 * same either way. */
typedef struct {
    wh_tensor weight;
    size_t row_start, row_end;
    const float* x_dev; /* cols floats */
    float* y_dev;       /* row_end - row_start floats */
} wh_gemv_desc;
int wh_fp8_gemv_batch_async(wh_ctx* ctx, const wh_gemv_desc* descs, size_t n);

/* Device-pointer variant of wh_fp8_gemv_multi (gemv_fp8_e4m3_ue8m0_rows_multi,
 * E/compute.rs:6384-6577): n f32 inputs at x_dev + i * x_stride, outputs at
 * y_dev + i * y_stride, each bit-identical to the single-input GEMV in the
 * same numerics mode.  With exact numerics off (wh_set_exact_numerics(ctx, 0)) and at least
 * wh_set_fp8_mfma_min inputs, tensors of a multiple of 256 columns in
 * 128-column scale groups, scale rows of a power of two >= 16 rows and
 * row_start % 16 == 0 run on bf16 MFMA instead: each weight byte is read once
 * for all inputs, the weights are the reference's values exactly and each
 * input is split exactly into three bf16 parts, so every product is exact
 * and the outputs differ from the reference kernel's by fp32 accumulation
 * order only (within 1e-5 * ||w_row||_2 * ||x||_2). */
int wh_fp8_gemv_multi_async(wh_ctx* ctx, wh_tensor w, size_t row_start, size_t row_end, const float* x_dev, size_t n,
                            size_t x_stride, float* y_dev, size_t y_stride);

/* Two wh_fp8_gemv_multi_async calls on the same n inputs, in order: rows
 * [row_start0, row_end0) of w0 into y0_dev and rows [row_start1, row_end1) of
 * w1 into y1_dev (wq_a and wkv of a batch of decode positions; the reference
 * calls rows_multi once for each, E/compute.rs:4005-4013, 6384-6577).
 * Results are those of the two calls; when both take the MFMA path with the
 * same k split, the tensors share width, scale format, rows per scale row and
 * the special-code flag, and neither output overlaps the inputs or the other
 * output, they go out as one launch. */
int wh_fp8_gemv_multi_pair_async(wh_ctx* ctx, wh_tensor w0, size_t row_start0, size_t row_end0, float* y0_dev,
                                 size_t y0_stride, wh_tensor w1, size_t row_start1, size_t row_end1, float* y1_dev,
                                 size_t y1_stride, const float* x_dev, size_t n, size_t x_stride);

/* The reference's grouped batch projection, one rows_multi call per row group
 * with the group's own inputs (wo_a, E/compute.rs:4599-4622), as one call:
 * rows row_start + [g * group_rows, (g + 1) * group_rows) read input i of
 * group g at x_dev + i * x_stride + g * x_group_stride and write
 * y_dev + i * y_stride + (row - row_start).  Results are those of the
 * per-group wh_fp8_gemv_multi_async calls; on the MFMA path (as there, plus
 * group_rows a power of two >= 128) all groups go out as one launch. */
int wh_fp8_gemv_multi_groups_async(wh_ctx* ctx, wh_tensor w, size_t row_start, size_t row_end, size_t group_rows,
                                   const float* x_dev, size_t x_group_stride, size_t n, size_t x_stride, float* y_dev,
                                   size_t y_stride);

/* Multi-input FP8 GEMVs with at least min_inputs inputs take the MFMA path
 * when exact numerics are off (default 4; 0 = never).  No counterpart in the
 * reference. */
int wh_set_fp8_mfma_min(wh_ctx* ctx, uint32_t min_inputs);

/* Device-pointer FP8 GEMV (rows [row_start,row_end) of w, x_dev f32 or bf16). */
int wh_fp8_gemv_async(wh_ctx* ctx, wh_tensor w, size_t row_start, size_t row_end,
                      const float* x_dev, float* y_dev);

/* Deferred status of *_async calls (same as wh_synchronize). */
int wh_stream_status(wh_ctx* ctx);

/* Captured launch sequences, no counterpart in the reference (its decode step
 * runs on the CPU).  wh_graph_begin starts capturing the context stream: the
 * *_async calls the same thread makes until wh_graph_end are recorded, not
 * run, and wh_graph_end returns them as one HIP graph that wh_graph_launch
 * enqueues on the context stream (any number of times; failures surface in
 * wh_stream_status like those of the calls themselves).  A graph replays the
 * device addresses and host arguments it captured: inputs and outputs at the
 * same addresses, the same route lists, and the tensors and experts it reads
 * resident and unchanged until wh_graph_release.  Run the captured calls
 * once before capturing: a call that has to grow an internal buffer, or that
 * synchronizes (every call without _async, stores, releases), fails during
 * capture and wh_graph_end then returns an error (the context stays usable:
 * captures run on a stream of their own, which wh_stream returns meanwhile).
 * Buffers that grow after a capture are kept for the graphs until the last of
 * them is released.  Only the capturing thread may use the context between
 * begin and end. */
typedef uint64_t wh_graph;
int wh_graph_begin(wh_ctx* ctx);
int wh_graph_end(wh_ctx* ctx, wh_graph* out);
int wh_graph_launch(wh_ctx* ctx, wh_graph graph);
int wh_graph_release(wh_ctx* ctx, wh_graph graph);

/* Device buffers for the *_async entry points (the engine's resident
 * hidden-state buffers).  kind: 0 host->device, 1 device->host,
 * 2 device->device; wh_memcpy is ordered on the context stream and returns
 * when the copy is done. */
int wh_device_alloc(wh_ctx* ctx, size_t bytes, void** out);
int wh_device_free(wh_ctx* ctx, void* ptr);
int wh_memcpy(wh_ctx* ctx, void* dst, const void* src, size_t bytes, int kind);

/* Device timer on the context stream, the device counterpart of the
 * reference's ZC_PROF pass timers (E/server/generation.rs:2344-2351):
 * wh_timer_start records a HIP event on the stream; wh_timer_stop records a
 * second one, waits for it and returns the microseconds between the two -
 * the device time of everything enqueued in between. */
int wh_timer_start(wh_ctx* ctx);
int wh_timer_stop(wh_ctx* ctx, double* elapsed_us);

/* Measurement helper, no counterpart in the reference: the HBM read floor.
 * Times plain streaming-read launches of `bytes` (a multiple of 16) from
 * rotating windows of buf_dev (buf_bytes long, 16-byte aligned, at least one
 * 4 KiB-rounded window), `reps` back-to-back launches per grid size (256 to
 * 8192 workgroups of 256 threads) and loads in flight (4, 8, 16 x 16 B per
 * thread), on the library stream.  Writes the fastest mean microseconds per
 * launch with its grid and depth, and the per-launch cost of an empty
 * 1024 x 256 launch. */
int wh_probe_read_floor(wh_ctx* ctx, const void* buf_dev, size_t buf_bytes, size_t bytes, size_t reps,
                        double* best_us, uint32_t* best_grid, uint32_t* best_depth, double* empty_us);

/* Per-kernel timing of the routed-expert path, no counterpart in the
 * reference (the engine's ZC_PROF timers, E/server/generation.rs:2344-2351,
 * time whole passes on the CPU).  routes holds n_sets route lists of n_routes
 * entries each; every list must resolve to experts on the fast path.  Each
 * kernel stage (gate/up + SwiGLU, then down + routed sum) is launched iters
 * times back to back, cycling through the lists so that the weights come
 * from HBM, between two HIP events on the context stream.  us_per_launch[0]
 * and [1] receive the mean microseconds per launch of the two stages.  The
 * down stage reads whatever hidden vector the last gate/up launch left. */
int wh_profile_routed(wh_ctx* ctx, const wh_expert_route* routes, size_t n_routes, size_t n_sets,
                      const void* x_dev, int x_is_bf16, float* out_dev, size_t iters,
                      double* us_per_launch);
/* Measurement support, no counterpart in the reference: `iters` routed-expert
 * tokens enqueued by one call, each token's gate/up then down, in the current
 * numerics mode; token i takes route set i % n_sets (n_routes entries each),
 * input row i % n_sets of x_dev (rows x_stride bytes apart, a multiple of 16)
 * and output row i % n_sets of out_dev (hidden floats).  mode 0: a host loop
 * of launches; 1: the same launches captured once into a HIP graph (kernel
 * nodes only) and replayed.  *us_per_token: mean between HIP events on the
 * context stream around the timed launches (the graph's second replay). */
int wh_profile_token_pipeline(wh_ctx* ctx, const wh_expert_route* routes, size_t n_routes, size_t n_sets,
                              const void* x_dev, int x_is_bf16, size_t x_stride, float* out_dev, size_t iters,
                              int mode, double* us_per_token);

/* Test support, no counterpart in the reference: evaluates the device libm
 * emulation on n values.  fn 0: silu(x) = x / (1 + expf(-x)) for x <= 10;
 * fn 1: expf(x); fn 2: the act-quant block scale
 * exp2f(ceilf(log2f(max(x, 1e-4) / 448))) for finite x >= 0; fn 3: a plain
 * device copy out = in (n a multiple of 4) that calibrates HBM byte counters;
 * fn 4: the router's sqrt_softplus(x); fn 5: log1pf(x) for x >= 0; fn 6:
 * expf(x) for any x; fn 7 / 8: the act-quant (block 64) of the LDS-streaming
 * token kernels for bf16 / f32 inputs (n a multiple of 64, finite values;
 * fn 7's inputs must be bf16 values), dequantized. */
int wh_debug_eval(wh_ctx* ctx, int fn, const float* in, float* out, size_t n);

/* ------------------------------------------------------------------
 * MLA attention glue at decode (compute_deepseek_v4_mla_attention,
 * E/compute.rs:3924-4293): the non-GEMV steps between the FP8 projections,
 * bit-identical to the reference's f32 arithmetic (sequential sums, separate
 * roundings, glibc-exact expf / sinf / cosf, the block-64 act-quant).
 * Positions must be below 2^24 (WH_UNSUPPORTED otherwise).
 * ------------------------------------------------------------------ */

/* YarnRope (E/compute.rs:2558-2572). */
typedef struct {
    float factor, beta_fast, beta_slow;
    size_t original_seq_len;
} wh_yarn;

/* rope_inv_freqs (E/compute.rs:2591-2620), on the host with the platform
 * libm as the reference computes it: rope_dim / 2 values; yarn NULL = plain
 * theta^(-2i/dim). */
int wh_rope_inv_freqs(size_t rope_dim, float theta, const wh_yarn* yarn, float* out, size_t out_len);
/* deepseek_rope_for_layer (E/compute.rs:2575-2586): theta 160000 with
 * DEEPSEEK_V4_YARN on layers with a compress ratio, else 10000 without. */
int wh_deepseek_rope_for_layer(uint32_t physical_layer, float* theta, wh_yarn* yarn, int* has_yarn);

/* rms_norm_in_place (E/compute.rs:7110-7122) of each of `rows` rows of n
 * values (weight_bf16_dev NULL), or apply_weighted_rms_norm
 * (E/compute.rs:3077-3107) with a bf16 weight of n values; eps 1e-6.
 * out_dev may equal x_dev.  n <= 4096.  With exact numerics (the default)
 * the sum of squares runs in the reference's order, bit-identical; with
 * exact numerics off it is a fixed tree (the same value up to rounding,
 * reproducible), as are the norms inside wh_mla_attention_decode_async. */
int wh_rms_norm_async(wh_ctx* ctx, const float* x_dev, float* out_dev, size_t rows, size_t n,
                      const uint16_t* weight_bf16_dev);

/* apply_rope_interleaved_with_freqs (E/compute.rs:2623-2649) on
 * values[r * row_stride + offset .. + 2 * pairs) of each row r, at
 * `position`, with inverse frequencies inv_freqs_dev[pairs]; inverse != 0
 * rotates back.  offset + 2 * pairs > row_stride -> WH_INVALID_SHAPE
 * ("RoPE input shorter than dim").  row_stride <= 4096. */
int wh_rope_async(wh_ctx* ctx, float* values_dev, size_t rows, size_t row_stride, size_t offset,
                  const float* inv_freqs_dev, size_t pairs, size_t position, int inverse);

/* Device-pointer fp8_act_quant_dequant_in_place (E/compute.rs:2504-2521). */
int wh_act_quant_dequant_async(wh_ctx* ctx, float* values_dev, size_t n, size_t block_size);

/* The window softmax of the MLA layer (E/compute.rs:4106-4197) for one
 * decode position: per head h the keys are the n_window rows at window_dev
 * (row stride window_stride; the KV cache from the window start) then the
 * n_comp compressed rows (head_dim apart); score = (q . key in order) *
 * head_dim^-0.5, softmax against the largest score with the optional sink
 * logit sink_dev[h] in the denominator, out = sum of weight * key in key
 * order, divided by the denominator when positive, then the inverse RoPE of
 * the rope dims [nope_dim, nope_dim + 2 pairs) at token_pos.  scores_dev:
 * heads * (n_window + n_comp) floats of scratch.  head_dim a multiple of 64,
 * at most 1024; at most 2048 keys; window_dev and comp_dev 16-byte aligned
 * and window_stride a multiple of 4 (WH_INVALID_ARGUMENT otherwise). */
int wh_window_attention_async(wh_ctx* ctx, const float* q_dev, size_t heads, size_t head_dim, size_t nope_dim,
                              const float* window_dev, size_t n_window, size_t window_stride, const float* comp_dev,
                              size_t n_comp, const float* sink_dev, const float* inv_freqs_dev, size_t pairs,
                              size_t token_pos, float* scores_dev, float* out_dev);

/* One decode MLA attention layer (compute_deepseek_v4_mla_attention,
 * E/compute.rs:3924-4293) with resident FP8 projections: act-quant x; q_lora
 * = wq_a x; q norm (weighted if q_norm_bf16, else plain) + act-quant; q =
 * wq_b q_lora; per-head RMS norm and RoPE; kv = wkv x; kv norm, RoPE,
 * act-quant of the non-rope dims, stored as the KV cache row of token_pos;
 * the window softmax over the cached rows [max(0, token_pos - 127),
 * token_pos] and the n_comp compressed rows the caller passes (the
 * compressor's visible blocks, E/compute.rs:4087-4100); act-quant; wo_a per
 * output group; act-quant; hidden = wo_b o_mid (in place).  RoPE theta and
 * YaRN follow physical_layer.  Shapes: wq_a [q_lora x hidden], wq_b
 * [heads*head_dim x q_lora], wkv [head_dim x hidden], wo_a [o_groups*o_lora
 * x heads*head_dim/o_groups], wo_b [hidden x o_groups*o_lora]; a mismatch
 * is WH_INVALID_SHAPE.  hidden_dev, kv_cache_dev and comp_dev 16-byte
 * aligned, kv_stride a multiple of 4. */
typedef struct {
    uint32_t physical_layer;
    size_t heads, nope_dim, rope_dim, o_groups, o_lora_rank;
    wh_tensor wq_a, wq_b, wkv, wo_a, wo_b;
    const uint16_t* q_norm_bf16;  /* device [q_lora] or NULL */
    const uint16_t* kv_norm_bf16; /* device [head_dim] or NULL */
    const float* sink;            /* device [heads] or NULL */
} wh_mla_layer;
int wh_mla_attention_decode_async(wh_ctx* ctx, const wh_mla_layer* layer, size_t token_pos, float* hidden_dev,
                                  float* kv_cache_dev, size_t kv_stride, size_t kv_capacity, const float* comp_dev,
                                  size_t n_comp);

/* The batched MLA attention of prefill and MTP verify
 * (compute_deepseek_v4_mla_attention_batch, E/compute.rs:4307-4641) over
 * npos positions in ascending order (hidden_dev [npos x hidden] in place,
 * their KV cache rows written): the projections run over all positions at
 * once (gemv_fp8_e4m3_ue8m0_rows_multi, each input bit-identical to the
 * single-input kernels with exact numerics), the norms, RoPE and cache rows
 * per position, then each position's window softmax over the cache rows up
 * to its own and its n_comp[i] compressed rows at comp_dev[i] (host arrays
 * of npos entries, or NULL for none).  With exact numerics the outputs
 * equal npos calls of wh_mla_attention_decode_async in position order. */
int wh_mla_attention_decode_batch_async(wh_ctx* ctx, const wh_mla_layer* layer, const size_t* positions, size_t npos,
                                        float* hidden_dev, float* kv_cache_dev, size_t kv_stride, size_t kv_capacity,
                                        const float* const* comp_dev, const size_t* n_comp);

/* ------------------------------------------------------------------
 * mHC hyper-connections (E/compute.rs:4945-5092), device pointers, f32.
 * hc copies of the hidden state form a stream of hc * hidden floats;
 * mix_hc = (2 + hc) * hc; hc <= 14.
 * ------------------------------------------------------------------ */

/* hc_split_sinkhorn_scalar (E/compute.rs:4945-5014): pre[hc] =
 * sigmoid(mixes * scale[0] + base) + eps, post[hc] = 2 sigmoid(mixes[hc..] *
 * scale[1] + base[hc..]), comb[hc][hc] = row softmax(mixes[2hc..] * scale[2]
 * + base[2hc..]) + eps, normalised by columns once and then by rows and
 * columns sinkhorn_iters - 1 more times.  Bit-identical to the reference
 * (glibc-exact expf, sums in order). */
int wh_hc_split_sinkhorn_async(wh_ctx* ctx, const float* mixes_dev, const float* scale_dev, const float* base_dev,
                               size_t hc, size_t sinkhorn_iters, float eps, float* pre_dev, float* post_dev,
                               float* comb_dev);

/* hc_pre_into (E/compute.rs:5016-5050): mixes[j] = (fn row j . x) *
 * 1 / sqrt(mean(x^2) + eps) for the mix_hc rows of fn_dev ([mix_hc][hc *
 * hidden]), then hc_split_sinkhorn, then y[d] = sum over i of pre[i] *
 * x[i * hidden + d].  post_dev[hc] and comb_dev[hc * hc] receive what
 * hc_post needs.  With exact numerics (the default) the dot products and
 * the sum of squares run in the reference's order, bit-identical; with
 * exact numerics off they are summed over many workgroups in a fixed tree
 * (same value up to rounding, reproducible), everything after them still
 * in the reference's order. */
int wh_hc_pre_async(wh_ctx* ctx, const float* fn_dev, const float* scale_dev, const float* base_dev, size_t hc,
                    size_t hidden, size_t sinkhorn_iters, float eps, const float* x_dev, float* y_dev,
                    float* post_dev, float* comb_dev);

/* hc_post_into (E/compute.rs:5055-5092): out[k * hidden + d] = post[k] *
 * y[d] + sum over i (in order) of comb[k * hc + i] * residual[i * hidden +
 * d].  Bit-identical to the reference. */
int wh_hc_post_async(wh_ctx* ctx, const float* y_dev, const float* residual_dev, const float* post_dev,
                     const float* comb_dev, float* out_dev, size_t hc, size_t hidden);

/* ------------------------------------------------------------------
 * One DeepSeek-V4 decode layer on the device: compute_layer_deepseek_mhc
 * (E/compute.rs:1448-1480) with the router between its two phases as the
 * engine runs them (E/server/generation.rs:719-836).  On the hc copies of
 * the hidden state at hidden_dev (hc * hidden floats, updated in place):
 *   attention sub-block (phase 1, E/compute.rs:1552-1605): y = hc_pre(hc_attn,
 *     hidden); y = rms_norm(y, attn_norm); y = MLA attention(y) (as
 *     wh_mla_attention_decode_async, with the KV cache arguments below);
 *     hidden' = hc_post(y, hidden);
 *   ffn input (E/compute.rs:1607-1630): g = rms_norm(hc_pre(hc_ffn, hidden'),
 *     ffn_norm);
 *   router (route_experts_from_dense_block, E/compute.rs:2129-2268) of
 *     layer_id on g, as wh_route_experts_async;
 *   MoE (phase 2, E/compute.rs:1641-1700): z = shared(g) + routed experts of
 *     layer_id on the router's list (wh_routed_and_shared_experts_dev_async);
 *     hidden = hc_post(z, hidden').
 * Every step is the kernel of its own entry point, so the layer is
 * bit-identical to the reference under exact numerics; with exact numerics
 * off the FP8 projections, the expert matvecs and hc_pre's sums take the
 * order-free kernels (the router keeps the reference order).  Nothing is
 * read back to the host: the whole layer can be captured (wh_graph_begin).
 * hidden_dev 16-byte aligned; the norm weights are bf16 (NULL: plain RMS
 * norm); available_dev / n_available as in wh_route_experts_async. */
typedef struct {
    size_t hc, hidden, sinkhorn_iters;
    float hc_eps;
    const float* hc_attn_fn;     /* device [(2 + hc) * hc][hc * hidden] */
    const float* hc_attn_scale;  /* device [3] */
    const float* hc_attn_base;   /* device [(2 + hc) * hc] */
    const float* hc_ffn_fn;
    const float* hc_ffn_scale;
    const float* hc_ffn_base;
    const uint16_t* attn_norm_bf16;  /* input_layernorm [hidden] or NULL */
    const uint16_t* ffn_norm_bf16;   /* post_attention_layernorm [hidden] or NULL */
    wh_mla_layer attn;
    uint32_t layer_id;           /* router and routed experts */
    size_t active;               /* experts per token */
    const uint32_t* available_dev;
    size_t n_available;
    wh_route_options route;
    uint32_t shared_layer, shared_expert;  /* WH_NO_SHARED_EXPERT: none */
} wh_mhc_layer;
int wh_deepseek_mhc_layer_async(wh_ctx* ctx, const wh_mhc_layer* layer, size_t token_pos, float* hidden_dev,
                                float* kv_cache_dev, size_t kv_stride, size_t kv_capacity, const float* comp_dev,
                                size_t n_comp);

/* The batched layer of prefill and MTP verify (E/server/generation.rs:
 * 2437-2590), replacing compute_layer_deepseek_mhc_phase1_batch
 * (E/compute.rs:4649-4750), the per-position router and
 * finish_layer_deepseek_mhc_phase2_batch (E/compute.rs:1817-1870):
 * hidden_dev holds npos states of hc * hidden floats at ascending positions.
 *   phase 1: per position y = rms_norm(hc_pre(hc_attn, hidden), attn_norm);
 *     the attention of all positions as wh_mla_attention_decode_batch_async;
 *     per position hidden' = hc_post(y, hidden) and g = rms_norm(hc_pre(
 *     hc_ffn, hidden'), ffn_norm);
 *   the router per position on its g (wh_route_experts_async);
 *   the MoE of the batch as wh_moe_batch_async: the union of the selected
 *     experts in ascending id, each position's router weights divided by
 *     their sum (the reference's batch path, E/server/generation.rs:
 *     2487-2506, which renormalises the route_scale'd weights to 1), plus the
 *     shared expert; hidden = hc_post(z, hidden').
 * token_ids: each position's token for a hash layer's row (the reference
 * passes each item's token id, E/server/generation.rs:2462-2474), or NULL
 * for layer->route.hash_token_id at every position.
 * With exact numerics every position is bit-identical to the reference's
 * batch path.  WH_UNSUPPORTED when an availability list has fewer than
 * `active` entries (the batch MoE takes `active` routes per position).  At
 * the model's expert shapes nothing is read back to the host. */
int wh_deepseek_mhc_layer_batch_async(wh_ctx* ctx, const wh_mhc_layer* layer, const size_t* positions, size_t npos,
                                      float* hidden_dev, float* kv_cache_dev, size_t kv_stride, size_t kv_capacity,
                                      const float* const* comp_dev, const size_t* n_comp, const int64_t* token_ids);

#ifdef __cplusplus
}
#endif
#endif /* WOHPER_HIP_H */
