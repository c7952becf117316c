/*
 * sox_backend.h - the HIP backend behind SimdOnnx's backend surface, as a C ABI.
 *
 * It mirrors the reference's three-class GPU backend surface and its extension hook:
 *   HipBackend          <- VkBackend (Backends/Vulkan/VkBackend.cs:11-267): device, Default /
 *                          TryGetDefault, IsLost, graph building
 *   HipGraphModel       <- VkGraphModel (Backends/Vulkan/VkGraph.cs:44-1233): const packing and
 *                          upload, one Emit per ExecNode producing dispatch records
 *   HipInferenceSession <- VkInferenceSession (Backends/Vulkan/VkSession.cs:63-571): one arena
 *                          slab, mapped fp32 staging, Run / Submit / Wait, DebugProfile
 *   ext emit hook       <- ExtOp.EmitVulkan + VkGraphModel.Dispatch (Engine/Extensions.cs:41-50,
 *                          VkGraph.cs:1117-1123)
 * The plan a caller hands over is the reference's ExecPlan (Engine/ExecPlan.cs:235-317) as the
 * unchanged GraphCompiler produced it for PlanTarget.Hip: values (shape, physical layout, arena
 * buffer or const data), nodes (ExecOp + value ids + the op's parameter record) and the arena plan.
 * All status codes are those of sox_hip.h.
 */
#ifndef SOX_BACKEND_H
#define SOX_BACKEND_H
#include <stddef.h>
#include <stdint.h>

#include "sox_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct sox_plan sox_plan;
typedef struct sox_backend sox_backend;
typedef struct sox_graph sox_graph;
typedef struct sox_session sox_session;

/* ExecOp, numbered as Engine/ExecPlan.cs:4-40. */
enum sox_exec_op {
    SOX_OP_CONV = 0, SOX_OP_MAXPOOL = 1, SOX_OP_ELEMENTWISE = 2, SOX_OP_RELU = 3, SOX_OP_SIGMOID = 4,
    SOX_OP_ERF = 5, SOX_OP_GELU = 6, SOX_OP_LAYERNORM = 7, SOX_OP_GEMM = 8, SOX_OP_RESIZE_BILINEAR = 9,
    SOX_OP_PAD = 10, SOX_OP_TRANSPOSE = 11, SOX_OP_SLICE = 12, SOX_OP_CONCAT = 13, SOX_OP_COPY = 14,
    SOX_OP_HARD_SIGMOID = 15, SOX_OP_GLOBAL_AVG_POOL = 16, SOX_OP_CONV_TRANSPOSE = 17, SOX_OP_RESIZE_NEAREST = 18,
    SOX_OP_MATMUL = 19, SOX_OP_SOFTMAX = 20, SOX_OP_REDUCE_MEAN = 21, SOX_OP_SQRT = 22, SOX_OP_AVGPOOL = 23,
    SOX_OP_HARDSWISH = 24, SOX_OP_SWISH = 25, SOX_OP_EXT = 26, SOX_OP_CHANNEL_GATE = 27, SOX_OP_ATTENTION = 28,
    SOX_OP_LEAKY_RELU = 29, SOX_OP_TANH = 30, SOX_OP_CLIP = 31, SOX_OP_DEPTH_TO_SPACE = 32, SOX_OP_SPACE_TO_DEPTH = 33
};

/* Parameter records (Engine/ExecPlan.cs:50-199), value ids -1 = none. */
typedef struct sox_conv_p {          /* ConvP :50-65 */
    int32_t pads[4];                 /* top, left, bottom, right */
    int32_t strides[2], dilations[2], kernel[2];
    int32_t group, act, pad_mode;    /* pad_mode: 0 constant, 1 reflect */
    float pad_value;
    int32_t bias_value, add_value;
    int32_t has_pool;                /* ConvP.Pool: fused 2x2/2 max pool, Out[0] is the pooled tensor */
    int32_t pool_kernel[2], pool_strides[2], pool_pads[4];
    int32_t pool_relu;
} sox_conv_p;

typedef struct sox_pool_p {          /* PoolP :67-74 */
    int32_t kernel[2], strides[2], pads[4];
    int32_t fuse_relu, count_include_pad;
} sox_pool_p;

typedef struct sox_ew_p { int32_t op, act; } sox_ew_p;                      /* EwP :76-80 */
typedef struct sox_ln_p { float eps; } sox_ln_p;                            /* LnP :82-85 */
typedef struct sox_gemm_p { int32_t trans_b, bias_value, act; } sox_gemm_p; /* GemmP :87-93 */
typedef struct sox_hard_sigmoid_p { float alpha, beta; } sox_hard_sigmoid_p; /* :103-106 */
typedef struct sox_convt_p { int32_t kernel[2]; int32_t bias_value, act; } sox_convt_p; /* ConvTP :108-114 */
typedef struct sox_resize_nearest_p { float scales[4]; int32_t add_relu; } sox_resize_nearest_p; /* :116-121 */
typedef struct sox_concat_p { int32_t axis; } sox_concat_p;                 /* ConcatP :196-199 */
typedef struct sox_channel_gate_p {                                          /* ChannelGateP :151-158 */
    int32_t b1, b2, act1, hard;
    float alpha, beta, offset;
} sox_channel_gate_p;
typedef struct sox_attention_p {                                             /* AttentionP :166-174 */
    float scale;
    int32_t dims[3][4];              /* per operand: logical axes holding (n, h, t|s, d), -1 = size 1 */
    int32_t fix_axis[3], fix_index[3];
    int32_t out_layout[4];           /* physical order of the [n,h,t,d] output; all -1 = identity */
} sox_attention_p;

typedef struct sox_resize_p {                                                /* ResizeP :95-101 */
    float scales[4];                 /* only [.., sh, sw] used */
    int32_t fuse_relu, add_relu;     /* relu on the resized value / on the addend In[1] */
} sox_resize_p;
typedef struct sox_pad_p {                                                   /* PadP :176-181 */
    int32_t rank;
    int32_t pads[12];                /* [2*rank] logical begin.., end.. */
    int32_t mode;                    /* PadMode: 0 constant, 1 reflect */
    float value;
} sox_pad_p;
typedef struct sox_transpose_p { int32_t rank; int32_t perm[6]; } sox_transpose_p; /* TransposeP :183-186 (physical perm) */
typedef struct sox_slice_p {                                                 /* SliceP :188-194 (physical axes, resolved starts) */
    int32_t naxes;
    int32_t starts[6], ends[6], axes[6], steps[6];
} sox_slice_p;
typedef struct sox_leaky_relu_p { float alpha; } sox_leaky_relu_p;           /* LeakyReluP :123-126 */
typedef struct sox_tanh_p { float in_scale, out_scale; } sox_tanh_p;         /* TanhP :129-133 */
typedef struct sox_clip_p { float min, max; } sox_clip_p;                    /* ClipP :134-138 */
typedef struct sox_depth_to_space_p { int32_t block, crd; } sox_depth_to_space_p; /* DepthToSpaceP :139-145 */

/* Records of the built-in extension ops (ExecOp.Ext with these names; Engine/Fusions/SafeDivOp.cs, ChannelShiftOp.cs, UpHeadOp.cs). */
typedef struct sox_safediv_p { float eps, lo, hi; } sox_safediv_p;      /* SafeDivP, SafeDivOp.cs:9-13 */
typedef struct sox_shift_p {                                               /* ShiftP, ChannelShiftOp.cs:9-14 */
    int32_t axis;                    /* logical spatial axis: 2 = H, 3 = W */
    int32_t ngroups;                 /* <= 5 */
    int32_t group_ends[5], offsets[5];
} sox_shift_p;
typedef struct sox_uphead_p {                                              /* UpHeadP, UpHeadOp.cs:15-32 */
    float scales[4];
    int32_t resize_relu, skip_relu, act;
    int32_t has_skip_conv;           /* In[1] is the skip conv's input (UpHeadP.SkipConv) */
    sox_conv_p skip_conv;
    int32_t skip_w, skip_b;          /* the skip conv's weight / bias value ids (-1 none) */
} sox_uphead_p;

/* ---- plan (ExecPlan) ---- */
int sox_plan_create(sox_plan** plan);
void sox_plan_destroy(sox_plan* plan);
/* CValue (ExecPlan.cs:202-220). shape = logical dims; layout = physical order (layout[i] = the
 * logical dim stored at physical position i; NULL = identity); buf >= 0: activation buffer id,
 * else a const whose nfloats floats are copied. */
int sox_plan_add_value(sox_plan* plan, const int32_t* shape, int32_t rank, const int32_t* layout, int32_t buf,
                       const float* floats, int64_t nfloats, const char* name, int32_t* id);
/* ExecNode (ExecPlan.cs:235-276); params is the op's record above (bytes copied). Ext nodes pass
 * the extension op's registered name as `ext_name` and an opaque params blob. */
int sox_plan_add_node(sox_plan* plan, int32_t op, const int32_t* in, int32_t nin, const int32_t* out, int32_t nout,
                      const void* params, size_t params_bytes, const char* ext_name, int32_t* id);
/* ExecPlan.BufOffset / ArenaFloats (ExecPlan.cs:283-285): offsets in elements. */
int sox_plan_set_arena(sox_plan* plan, const int64_t* buf_offset, int32_t nbuf, int64_t arena_floats);
int sox_plan_set_io(sox_plan* plan, const int32_t* inputs, int32_t ninputs, int32_t output);

/* ---- backend (VkBackend) ---- */
int sox_backend_default(sox_backend** backend);   /* Default: device 0, re-created after a device loss */
int sox_backend_info(sox_backend* backend, sox_device_info* info);
int sox_backend_is_lost(sox_backend* backend);
/* No counterpart in the reference (its analogue is the Vulkan validation layer, VkDevice.cs:176): a
 * backend that touches no device. Graphs built on it run every graph-creation step (the rewrites,
 * the arena changes, const packing, kernel choice against the embedded code objects' symbol tables)
 * and can be inspected (dispatch_*, value_place, const/arena bytes), but sessions, CTC heads, image
 * sessions, unit runners and extension code objects need a device and return SOX_E_UNSUPPORTED.
 * info = NULL describes an MI355X (gfx950, 256 CUs, 8 XCDs). For host-only checks (sanitizer builds,
 * CI without a GPU). */
int sox_backend_create_offline(const sox_device_info* info, sox_backend** backend);
/* Frees an offline backend (the device backend of sox_backend_default lives for the process). */
void sox_backend_destroy(sox_backend* backend);
/* Loads an extension's code object (an embedded resource of its owner, ShaderResources.Open). */
int sox_backend_load_module(sox_backend* backend, const void* image, size_t bytes, void** module);

/* ---- extension ops (ExtOp.EmitVulkan analogue) ---- */
typedef struct sox_bind { int32_t slot; int32_t pad_; uint64_t offset, size; } sox_bind; /* VkBind, VkGraph.cs:12-21 */
/* SOX_SLOT_SYNC: the session's cross-workgroup counters (zeroed once, back at 0 after every launch that
 * uses them; no counterpart in the reference, whose SE gate is a dispatch of its own) */
enum { SOX_SLOT_ARENA = 0, SOX_SLOT_CONSTS = 1, SOX_SLOT_DUMMY = 2, SOX_SLOT_SYNC = 3 };
/* ConstKind (Engine/Extensions.cs:144-159) as an id. */
enum { SOX_CK_RAW = 0, SOX_CK_F32 = 1, SOX_CK_CONVWT = 2, SOX_CK_GEMMNK = 3, SOX_CK_DWW = 4, SOX_CK_CONVTW = 5,
       SOX_CK_F32T = 7 /* fp32, rank-2 view [a][b...] transposed to [b...][a] */ };
typedef int (*sox_ext_emit_fn)(void* user, sox_graph* graph, int32_t node);
typedef int (*sox_ext_consts_fn)(void* user, const sox_plan* plan, int32_t node, int32_t* values, int32_t* kinds,
                                 int32_t cap); /* GpuConsts: returns the count written */
int sox_backend_register_ext(sox_backend* backend, const char* name, sox_ext_emit_fn emit, sox_ext_consts_fn consts,
                             void* user);
/* Inside an emit callback: Bind(valueId, kind) and Dispatch(n, kernel, binds, params, grid). The
 * kernarg block is the binds' device addresses (8 bytes each, in order) followed by params. */
int sox_graph_bind(sox_graph* graph, int32_t value, int32_t const_kind, sox_bind* out);
int sox_graph_scratch(sox_graph* graph, uint64_t bytes, sox_bind* out);
int sox_graph_dispatch(sox_graph* graph, int32_t node, void* module, const char* kernel, const sox_bind* binds,
                       int32_t nbinds, const void* params, size_t params_bytes, const uint32_t grid[3],
                       const uint32_t block[3], uint32_t lds_bytes);
int sox_graph_node_info(sox_graph* graph, int32_t node, int32_t* op, const void** params, size_t* params_bytes);
/* ExecNode.In / ExecNode.Out (ExecPlan.cs:235-276) of a node: up to in_cap / out_cap value ids are
 * written, *nin / *nout receive the full counts. */
int sox_graph_node_values(sox_graph* graph, int32_t node, int32_t* in, int32_t in_cap, int32_t* nin, int32_t* out,
                          int32_t out_cap, int32_t* nout);
int sox_graph_value_shape(sox_graph* graph, int32_t value, int32_t* phys_shape, int32_t cap, int32_t* rank);
int sox_graph_is_f16(sox_graph* graph); /* the storage mode: SOX_STORAGE_F32 / _F16 / _BF16 (0 / 1 / 2) */

/* ---- graph model (VkGraphModel) ---- */
/* Builds the dispatch list of a plan. f16 = the storage mode: SOX_STORAGE_F16 (1) = fp16 activation /
 * weight storage with fp32 math (the reference GPU contract, Backends/Vulkan/VkGraph.cs:33-43),
 * SOX_STORAGE_BF16 (2) = the same with bfloat16 storage (rounded to nearest even; bf16 matrix-core
 * instructions with fp32 accumulation; no reference counterpart), SOX_STORAGE_F32 (0) = fp32. */
enum { SOX_STORAGE_F32 = 0, SOX_STORAGE_F16 = 1, SOX_STORAGE_BF16 = 2 };
int sox_graph_create(sox_backend* backend, const sox_plan* plan, int32_t f16, sox_graph** graph);
void sox_graph_release(sox_graph* graph);
int sox_graph_dispatch_count(sox_graph* graph);
int sox_graph_dispatch_info(sox_graph* graph, int32_t index, char* name, size_t name_cap, uint32_t grid[3],
                            int32_t* node);
/* The code object function dispatch `index` launches (its tiling, e.g. sox_gemm_f16_256x192_w8k64s2),
 * next to the op label of sox_graph_dispatch_info: what a per-kernel profiler trace names it. */
int sox_graph_dispatch_kernel(sox_graph* graph, int32_t index, char* kernel, size_t kernel_cap);
/* The arena and const bindings dispatch `index` is patched with, in kernarg order (VkDispatch.Binds,
 * VkGraph.cs:24-31): up to cap written, *n = the count. */
int sox_graph_dispatch_binds(sox_graph* graph, int32_t index, sox_bind* binds, int32_t cap, int32_t* n);
/* The place of activation `value` in a session's slab after the graph-creation rewrites (BufOffset x
 * element size, VkGraph.cs:362-368): byte offset and size. A value moved to a buffer of its own moves
 * with its views, which report the same offset. */
int sox_graph_value_place(sox_graph* graph, int32_t value, uint64_t* offset, uint64_t* bytes);
uint64_t sox_graph_arena_bytes(sox_graph* graph);
uint64_t sox_graph_const_bytes(sox_graph* graph);
/* Bytes of cross-workgroup counters (SOX_SLOT_SYNC) each session of the graph holds (0: none). */
uint64_t sox_graph_sync_bytes(sox_graph* graph);
/* Last build error text (NotSupportedException message analogue). */
const char* sox_last_error(void);

/* ---- session (VkInferenceSession); not thread-safe: one per thread ---- */
int sox_session_create(sox_graph* graph, sox_session** session);
void sox_session_destroy(sox_session* session);

/* ---- shared session buffers (VkBufferPool / VkSessionBuffers, Backends/Vulkan/VkBatch.cs:6-25,
 * VkSession.cs:10-55) ----
 * The arena slab, device staging and pinned fp32 input / output staging of the sessions of one owner
 * that run one at a time (one shape-varying OCR stage): each session then costs only its dispatch
 * list, and only the largest session's memory is held. The buffers grow (to the need, and by at least
 * half again) when a session needs more; growing makes every session created on the pool before it
 * stale. Borrowing sessions enqueue on the pool's one stream, so their runs never overlap on the
 * device; the host staging is shared, so write a session's input only after the previous session's
 * Wait. Not thread-safe. */
typedef struct sox_buffer_pool sox_buffer_pool;
int sox_buffer_pool_create(sox_backend* backend, sox_buffer_pool** pool);   /* VkBackend.CreateBufferPool (VkBackend.cs:220) */
/* VkBufferPool.Dispose: the buffers are freed with the last session that borrows them. */
void sox_buffer_pool_destroy(sox_buffer_pool* pool);
/* The pool's arena slab size and generation (bumped by each growth). */
int sox_buffer_pool_info(sox_buffer_pool* pool, uint64_t* arena_bytes, int32_t* generation);
/* NewSession(model, shape, options, pool) (VkBackend.cs:205-216): a session on the pool's buffers. */
int sox_session_create_pooled(sox_graph* graph, sox_buffer_pool* pool, sox_session** session);
/* IsStale (VkSession.cs:178-180): 1 once another session on the same pool grew its buffers. A stale
 * session cannot run: run / submit / time / profile / read_value / value_ptr / input / output return
 * SOX_E_INVALID with a message (sox_last_error); destroy it and create it again. */
int sox_session_is_stale(sox_session* session);
/* Mapped fp32 staging of graph input `index` / the output, in the plan's physical layout. */
int sox_session_input(sox_session* session, int32_t index, float** host, int64_t* count);
int sox_session_output(sox_session* session, float** host, int64_t* count);
/* Run = Submit + Wait. */
int sox_session_run(sox_session* session);
int sox_session_submit(sox_session* session);
int sox_session_wait(sox_session* session);
/* Replay the dispatch sequence from a captured HIP graph (1) or launch it node by node (0). While a
 * rocprofiler-sdk tool (rocprofv3) is loaded into the process, replay stays off (one note on stderr):
 * captured replay under its kernel tracer has crashed the host process. */
int sox_session_set_replay(sox_session* session, int32_t on);
/* 1 when the session replays a captured HIP graph, 0 when it launches node by node. */
int sox_session_is_replaying(sox_session* session);
/* Device-side timing with HIP events on the session stream: `iters` back-to-back enqueues of the
 * dispatch list (flags bit0: include the staging copies/conversions), total ms. */
enum { SOX_RUN_STAGING = 1, SOX_RUN_DISPATCHES = 2 };
int sox_session_time(sox_session* session, int32_t iters, int32_t flags, float* total_ms);
/* DebugProfile (VkSession.cs:413-490): per-dispatch device ms, min over `reps` runs. */
int sox_session_profile(sox_session* session, int32_t reps, float* ms, int32_t cap);
/* Debug read of any arena value as fp32 (node-by-node bisecting, VkDebugTests analogue). */
int sox_session_read_value(sox_session* session, int32_t value, float* host, int64_t count);
/* Device address of an arena value (advanced callers / tests). */
int sox_session_value_ptr(sox_session* session, int32_t value, void** dev);
void* sox_session_stream(sox_session* session);

/* ---- CTC head (CtcProjection, Decoding/CtcProjection.cs:12-75) ----
 * The class projection of a CTC head fused with the per-row argmax and the winner's softmax
 * probability, run on the device over a session's features so the [rows, classes] logits are never
 * stored or copied home. Create packs the weights once (fp16, column-major per class, as the GPU
 * const contract rounds them) and keeps them on the device; one object serves any number of sessions
 * (calls on one object serialize on its lock). */
typedef struct sox_ctc sox_ctc;
/* weights: row-major [inner][columns] (an ONNX MatMul's B); bias: [columns] or NULL. */
int sox_ctc_create(sox_backend* backend, const float* weights, const float* bias, int32_t inner, int32_t columns,
                   sox_ctc** ctc);
void sox_ctc_destroy(sox_ctc* ctc);
/* IsFused (CtcProjection.cs:41-42): 1 when the fused kernel serves this head (inner >= 64,
 * columns >= 1024, as MatMul.CanFuseArgMax; on the GPU also inner % 16 == 0 and inner <= 256). */
int sox_ctc_is_fused(sox_ctc* ctc);
/* ArgMax (CtcProjection.cs:44-58) over the activation `feature_value` of a session of an fp16 graph
 * ([batch * rows, inner], after sox_session_run / _wait): indices[r] = the largest logit's column
 * (ties keep the first), probabilities[r] = its softmax probability in (0, 1]. Runs on the
 * session's stream and returns when the host arrays are written. SOX_E_UNSUPPORTED only when the
 * head is not fused (nothing written, the reference's false); SOX_E_INVALID for a non-finite logit
 * ("Recognizer output is invalid."), an fp32 session, a feature value that is not a dense
 * [batch * rows, inner] activation still intact after the run (a later node's output overlapping
 * it in the arena), or too many rows. */
int sox_ctc_argmax(sox_ctc* ctc, sox_session* session, int32_t feature_value, int32_t batch, int32_t rows,
                   int32_t* indices, float* probabilities);
/* No counterpart in the reference: sox_ctc_argmax for callers that cannot allocate (code under HIP
 * graph capture, a serving loop, a harness that forbids hipMalloc). The same kernels on the same
 * checks, but no allocation, no copy home and no wait: the work is enqueued on the session's stream
 * and d_indices / d_probabilities (device arrays of batch * rows) and *d_status (device int32: 0, or
 * 1 for a non-finite logit, the reference's "Recognizer output is invalid.") are written when the
 * stream gets there. The column-range partials (column ranges x batch x rows x 12 bytes) go to the
 * GPU's static scratch (sox_scratch, SOX_SCRATCH_BYTES); a larger call returns SOX_E_INVALID.
 * Every call on one GPU shares that scratch: calls are serialised on the host (any thread, any
 * CtcProjection) and each call's stream waits for the previous call's kernels, so eager calls on
 * different streams do not race. A call captured into a graph (the stream is capturing) is ordered
 * by the stream the graph is launched on only: replays must not overlap other users of the scratch. */
int sox_ctc_argmax_noalloc(sox_ctc* ctc, sox_session* session, int32_t feature_value, int32_t batch, int32_t rows,
                           int32_t* d_indices, float* d_probabilities, int32_t* d_status);

/* ---- image session (VkImageSession, Backends/Vulkan/VkImageSession.cs:7-297) ----
 * Image-to-image inference with the pixel conversions on the device, in the same stream as the model:
 * one upload of the bytes, the dispatches, one download. The model maps [1, 3, H, W] to [1, 3, H, W];
 * the caller passes the graph built for the image's tensor size (sox_image_session_tensor_size, the
 * AcquireGraph of the reference). Not thread-safe: one run at a time. */
typedef struct sox_image_session sox_image_session;
enum { SOX_PIX_BGR24 = 0, SOX_PIX_RGB24 = 1, SOX_PIX_BGRA32 = 2, SOX_PIX_RGBA32 = 3 }; /* PixelFormat */
/* lut: PixelNormalization.Table [3][256] (tensor channel c, byte value); rgb_order: Normalization.Order
 * == Rgb; output_scale: OutputScale; pad_multiple / pad_top_left: PadMultiple / Padding == TopLeft
 * (ImageSessionOptions.cs:15-50). */
int sox_image_session_create(sox_backend* backend, const float* lut, int32_t rgb_order, float output_scale,
                             int32_t pad_multiple, int32_t pad_top_left, sox_image_session** session);
void sox_image_session_destroy(sox_image_session* session);
/* ImageSessionOptions.Pads: the tensor height / width an image of this size runs at. */
int sox_image_session_tensor_size(sox_image_session* session, int32_t width, int32_t height, int32_t* tensor_h,
                                  int32_t* tensor_w);
/* Run (VkImageSession.cs:253-280): src rows src_stride bytes apart, dst the same format and size (rows
 * dst_stride apart; may be src). 4-byte formats keep each pixel's alpha. graph: a single-input fp16 or
 * fp32 graph whose input and output are [1, 3, tensor_h, tensor_w] in NHWC storage. */
int sox_image_session_run(sox_image_session* session, sox_graph* graph, const uint8_t* src, int32_t width,
                          int32_t height, int32_t src_stride, uint8_t* dst, int32_t dst_stride, int32_t format);

/* ---- unit runner (VkUnitRunner, Backends/Vulkan/VkUnitRunner.cs:5-337) ----
 * Several graph units per call (e.g. OCR line batches of different widths), re-recorded every run
 * instead of one session per shape. Each unit owns a region of one grow-only arena and of the fp32
 * host staging; the units of a wave are spread round-robin over `streams` HIP streams, so small units
 * run side by side instead of one after another, and each wave ends on one event per stream. Waves
 * are submitted back to back; a finished wave can be consumed while later ones still run. Not
 * thread-safe. */
typedef struct sox_unit_runner sox_unit_runner;
int sox_unit_runner_create(sox_backend* backend, int32_t streams, sox_unit_runner** runner);
void sox_unit_runner_destroy(sox_unit_runner* runner);
/* Clear (:42-49): drops the previous run's units (it must have been waited for). */
int sox_unit_runner_clear(sox_unit_runner* runner);
/* Add (:51-60): a unit over `graph` (the runner takes its own reference); its index. */
int sox_unit_runner_add(sox_unit_runner* runner, sox_graph* graph, int32_t* unit);
/* Cut (:70-75): ends the current wave (the units added so far that are not in a wave yet). */
int sox_unit_runner_cut(sox_unit_runner* runner);
int sox_unit_runner_waves(sox_unit_runner* runner);
int sox_unit_runner_wave_end(sox_unit_runner* runner, int32_t wave);
/* Input (:87-93): the unit's input window, pinned fp32 host memory in the plan's physical layout (the
 * first call after the last Add lays out the buffers). Output (:95-100): valid once its wave was
 * waited for, until the next Submit. */
int sox_unit_runner_input(sox_unit_runner* runner, int32_t unit, float** host, int64_t* count);
int sox_unit_runner_output(sox_unit_runner* runner, int32_t unit, float** host, int64_t* count);
/* Submit (:146-167): every wave (inputs must be written); Wait (:169-178): wave `wave` and every
 * earlier one. */
int sox_unit_runner_submit(sox_unit_runner* runner);
int sox_unit_runner_wait(sox_unit_runner* runner, int32_t wave);

#ifdef __cplusplus
}
#endif
#endif
