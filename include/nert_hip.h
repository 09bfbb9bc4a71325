/*
 * nert_hip.h -- C-ABI of the gfx950 (MI355X) device layer for NERT.
 *
 * Two levels:
 *  1. Node level: nert_hip_run_node() runs one row of the HIP kernel table
 *     from a plain-C node description (nert_abi.h). It is the C form of the
 *     reference seam call `HipDevice().kernels().find(op)(node, in, out)`
 *     (include/nert/device.hpp:30-31,53-57,96; executor call site
 *     src/executor.cpp:534). The C++ seam itself, `nert::HipDevice()`, is
 *     exported from the same library with the reference's C++ signature.
 *  2. Kernel level: one entry point per kernel family with plain pointers,
 *     sizes and a stream. Each replaces the compute of the reference rows it
 *     names (the oracle in src/kernels/, the reference HIP layer in src/hip/).
 *
 * Conventions: every function returns 0 on success and non-zero on failure,
 * with the message in nert_hip_last_error() (thread-local). Tensor pointers are
 * device pointers unless stated otherwise. `stream` is a hipStream_t; NULL
 * selects the layer's own stream, on which all seam rows and transfers run.
 * Kernel-level calls are asynchronous: they return once the work is queued.
 * Element types use the nert_dtype codes of nert_abi.h.
 */
#ifndef NERT_HIP_H
#define NERT_HIP_H

#include <stdint.h>

#include "nert_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------- runtime --- */

/* Selects device 0 and creates the layer stream; replaces EnsureDevice
 * (src/hip_device.cpp:33-44). Non-zero when no HIP device is usable. */
int nert_hip_init(void);
const char* nert_hip_last_error(void);
int nert_hip_device_count(int* count);

/* Device memory; replaces HIPAllocator (src/hip_device.cpp:46-68).
 * bytes <= 0 returns NULL. nert_hip_free(NULL) is a no-op. */
void* nert_hip_malloc(int64_t bytes);
int nert_hip_free(void* ptr);

/* Blocking transfers on the layer stream; replace HIPTransfer
 * (src/hip_device.cpp:70-89). bytes == 0 is a no-op. Pageable host buffers
 * of 1 MiB or more are staged through pinned bounce buffers (pieces of 1 MiB
 * growing to 4 MiB, 2 host threads, host memcpy overlapped with the DMA);
 * pinned host buffers and smaller copies go straight to the DMA engine.
 * NERT_HIP_STAGING=0 turns the staging off. */
int nert_hip_memcpy_h2d(void* dst, const void* src, int64_t bytes);
int nert_hip_memcpy_d2h(void* dst, const void* src, int64_t bytes);
/* Pinned (page-locked) host memory, for callers that keep their inputs and
 * outputs where the DMA engine reads them directly. bytes <= 0 returns NULL;
 * nert_hip_host_free(NULL) is a no-op. No reference counterpart: the
 * reference's Transfer takes whatever host pointer the caller holds
 * (src/hip_device.cpp:70-89). */
void* nert_hip_host_alloc(int64_t bytes);
int nert_hip_host_free(void* ptr);
/* Asynchronous device-to-device copy (Identity/Reshape/Flatten payloads). */
int nert_hip_memcpy_d2d(void* dst, const void* src, int64_t bytes, void* stream);

void* nert_hip_default_stream(void);
int nert_hip_stream_sync(void* stream);
void* nert_hip_event_create(void);
int nert_hip_event_record(void* event, void* stream);
/* Waits for `stop`, then writes the elapsed milliseconds start -> stop. */
int nert_hip_event_elapsed_ms(void* start, void* stop, float* ms);
int nert_hip_event_destroy(void* event);

/* HIP-graph capture of the layer stream. Everything queued on the layer
 * stream between begin and end (kernel launches of any rows, device-to-device
 * copies) becomes one replayable graph; rows that must read device memory on
 * the host (control operands without a host shadow) cannot be captured and
 * fail the capture, while data-dependent error checks are deferred (see
 * nert_hip_take_error_flags; begin clears the error word first, eagerly,
 * keeping bits raised before the capture for the next take).
 * Workspaces (split-K partials, TopK state, ...) must reach their size before
 * capture: run the sequence once eagerly first. A later eager call may still
 * grow a workspace; while any graph exec is alive the replaced buffer is kept
 * (not freed) until the last graph exec is destroyed, so replays never touch
 * freed memory. No reference counterpart: the reference executor launches
 * rows one by one (src/executor.cpp:480-535). */
int nert_hip_capture_begin(void);
int nert_hip_capture_end(void** graph_exec);
int nert_hip_graph_launch(void* graph_exec, void* stream);
int nert_hip_graph_destroy(void* graph_exec);

/* Reads (and clears when set) the device error word that rows with
 * data-dependent failures raise: bit 0 = integer division by zero,
 * bit 1 = index out of range. Synchronises `stream`. While `stream` is being
 * captured into a graph it reports 0 without reading: the flag stays raised
 * and the first call after a replay reports it. A caller that replays graphs
 * holding such rows calls this after the replay to see their errors. Bits
 * that were raised when a capture began (eager rows before it) are reported
 * by the next call too. */
int nert_hip_take_error_flags(int32_t* flags_out, void* stream);

/* Host shadows. nert_hip_memcpy_h2d keeps a host copy of every upload of at
 * most 64 KiB, keyed by device address, so rows read control operands
 * (shapes, axes, K, scales, pads, indices they validate) without a D2H round
 * trip. Writes through the node level (nert_hip_run_node, the HipDevice()
 * rows), nert_hip_memcpy_d2d and nert_hip_free drop the shadows they overlap.
 * The kernel-level entry points below do not: a C caller that writes a
 * buffer with one of them and then passes that buffer to nert_hip_run_node
 * as a control operand calls nert_hip_forget_host_shadow(buffer, bytes)
 * first, or the row reads the uploaded (stale) values. No reference
 * counterpart (the reference rows read control operands back with a
 * blocking D2H copy, e.g. src/hip/gather.cu:160). */
int nert_hip_forget_host_shadow(const void* ptr, int64_t bytes);

/* ---------------------------------------------------------- node level --- */

/* Runs one row of the HIP table on device tensors: the 73 rows that
 * nert::HipDevice().kernels().find answers for (the reference's op types), plus
 * the fused rows that nert_amd's runner emits (FusedConv, FusedMatMul,
 * FusedAddLayerNorm, FusedAttention; no counterpart in the reference, and not
 * found through the seam). Returns a nert_status;
 * on error `err` receives the row's message ("<Op> (node '<name>'): ...",
 * the reference convention, e.g. src/kernels/gemm.cpp:60). The row's work is
 * queued on the layer stream; results are visible after the next blocking
 * transfer or nert_hip_stream_sync(NULL). */
int nert_hip_run_node(const char* op_type, const char* node_name, int64_t schema_version,
                      const nert_attr_desc* attrs, int n_attrs, const nert_tensor_desc* inputs, int n_inputs,
                      const nert_tensor_desc* outputs, int n_outputs, char* err, int err_len);

/* 1 when nert_hip_run_node has a row for op_type: KernelTable::find != null,
 * or one of the four fused runner rows. */
int nert_hip_has_row(const char* op_type);

/* ------------------------------------------------------ GEMM on MFMA --- */

/* Y[M,N] = alpha * op(A) * op(B) + beta * C. A is [M,K] (trans_a = 0) or
 * [K,M]; B is [K,N] (trans_b = 0) or [N,K]; C is absent (c_rank = 0 or
 * c = NULL), [N] (c_rank = 1) or [M,N] (c_rank = 2).
 * Replaces Gemm: src/kernels/gemm.cpp:59-137, src/hip/gemm.cu:75-158. */
int nert_hip_gemm_f32(const float* a, const float* b, const float* c, float* y, int64_t m, int64_t n, int64_t k,
                      int trans_a, int trans_b, float alpha, float beta, int c_rank, void* stream);

/* Batched Y[b][M,N] = A[b][M,K] * B[b][K,N] with up to four broadcast batch
 * axes: batch b decomposes over batch_dims (row-major) and each operand
 * advances by its own per-axis element stride (0 = broadcast). Y is dense.
 * Replaces MatMul: src/kernels/mat_mul.cpp:79-169, src/hip/mat_mul.cu:86-193. */
int nert_hip_matmul_f32(const float* a, const float* b, float* y, int64_t m, int64_t n, int64_t k, int batch_rank,
                        const int64_t* batch_dims, const int64_t* a_batch_strides, const int64_t* b_batch_strides,
                        void* stream);

/* MatMul with its elementwise followers in the epilogue: Y = scale * (A B),
 * then + bias[n] (bias may be NULL), then for act == 1 the erf Gelu chain
 * Y = Y * (erf(Y / p[0]) + p[1]) * p[2] (act_params = p). Each operation
 * rounds like the separate Mul / Add / Div / Erf / Add / Mul rows, so the
 * result equals running them after nert_hip_matmul_f32 bit for bit.
 * No counterpart in the reference: it backs the runner's FusedMatMul row
 * (an internal row the runner creates from those chains). */
int nert_hip_matmul_fused_f32(const float* a, const float* b, const float* bias, float* y, int64_t m, int64_t n,
                              int64_t k, int batch_rank, const int64_t* batch_dims, const int64_t* a_batch_strides,
                              const int64_t* b_batch_strides, float scale, int act, const float* act_params,
                              void* stream);

/* Convolution geometry, lifted to three spatial axes (depth, height, width)
 * with unit leading extents for 1-D/2-D, as src/kernels/conv.cpp:233-249. */
typedef struct nert_conv_desc {
    int64_t batch, in_channels, out_channels, group;
    int64_t in[3];
    int64_t kernel[3];
    int64_t out[3];
    int64_t stride[3];
    int64_t dilation[3];
    int64_t pad[3]; /* leading pads; trailing pads are implied by out[] */
} nert_conv_desc;

/* NCHW (or NCDHW) implicit-GEMM convolution, optional bias [M].
 * Replaces Conv: src/kernels/conv.cpp:138-295, src/hip/conv.cu:159-338. */
int nert_hip_conv_f32(const float* x, const float* w, const float* bias, float* y, const nert_conv_desc* d,
                      void* stream);
/* The same convolution with an epilogue: y = act(conv + bias + residual),
 * residual (optional, NULL) laid out like y; act 0 is none, 1 Relu
 * (std::max(0, v)), 2 SiLU (v * Sigmoid(v), the Sigmoid row's 1/(1+exp(-v))
 * then the Mul row's product); other codes fail. Each step rounds as the
 * separate Conv, Add, Relu / Sigmoid and Mul rows do, so the result is
 * bit-identical to running them one after another. No reference counterpart:
 * the reference executor runs those rows separately (src/executor.cpp:480-535);
 * the runner in nert_amd fuses them through the FusedConv row. */
int nert_hip_conv_fused_f32(const float* x, const float* w, const float* bias, const float* residual, float* y,
                            const nert_conv_desc* d, int act, void* stream);
/* Two convolutions of one input in one launch: y = act(conv3x3(x, w) + bias
 * + residual) as nert_hip_conv_fused_f32 computes it, and y2 = conv1x1(x, w2)
 * + bias2 at the same stride with pad 0 (w2 [M][C]; bias2 optional, NULL).
 * `d` describes the 3x3 convolution, which must have pad 1, dilation 1 and
 * group 1; y2 has y's shape. The 1x1 reads exactly the 3x3's centre-tap
 * inputs (a ResNet block's first conv and its downsampling shortcut), so it
 * shares the 3x3's staged input. y is bit-identical to
 * nert_hip_conv_fused_f32 with the same kernel configuration; y2 differs
 * from nert_hip_conv_f32 of the 1x1 only in the order of its fp32 additions.
 * No reference counterpart: the reference runs the two Conv rows separately
 * (src/executor.cpp:480-535); nert_amd's runner pairs them through the
 * FusedConv row (six inputs, two outputs). */
int nert_hip_conv_pair_f32(const float* x, const float* w, const float* bias, const float* residual, float* y,
                           const float* w2, const float* bias2, float* y2, const nert_conv_desc* d, int act,
                           void* stream);
/* nert_hip_conv_fused_f32 (w2 NULL) or nert_hip_conv_pair_f32 (w2 set) with
 * the weights also given in the order the 3x3 LDS-patch kernel stores them,
 * for weights that stay fixed across calls (a model's initializers, packed
 * once): w_packed[m][b][t][j] = w[m][8 b + j][t] for output channel m,
 * channel block b < C/group/8, tap t < KD*KH*KW (row-major over the
 * kernel's axes) and j < 8; C/group must be a multiple of 8. That kernel
 * copies the packed rows to LDS with 16-byte stores instead of transposing
 * 4-byte ones; every other kernel reads w. Results are bit-identical to the
 * unpacked call with the same kernel configuration. No reference
 * counterpart: nert_amd's runner packs the 3x3 initializer weights and
 * passes them as the FusedConv row's seventh input. */
int nert_hip_conv_packed_f32(const float* x, const float* w, const float* w_packed, const float* bias,
                             const float* residual, float* y, const float* w2, const float* bias2, float* y2,
                             const nert_conv_desc* d, int act, void* stream);

/* ---------------------------------------------------------- elementwise --- */

enum nert_unary_op {
    NERT_UN_RELU = 0,   /* src/kernels/relu.cpp:51-53      std::max(0, x) */
    NERT_UN_SIGMOID,    /* src/kernels/sigmoid.cpp:52      1/(1+exp(-x)) */
    NERT_UN_TANH,       /* src/kernels/tanh.cpp */
    NERT_UN_EXP,        /* src/kernels/exp.cpp:48 */
    NERT_UN_LOG,        /* src/kernels/log.cpp */
    NERT_UN_SQRT,       /* src/kernels/sqrt.cpp:48 */
    NERT_UN_SIN,        /* src/kernels/sin.cpp */
    NERT_UN_COS,        /* src/kernels/cos.cpp */
    NERT_UN_FLOOR,      /* src/kernels/floor.cpp:48 */
    NERT_UN_ABS,        /* src/kernels/abs.cpp (f32, i64) */
    NERT_UN_NEG,        /* src/kernels/neg.cpp (f32, i64) */
    NERT_UN_SIGN,       /* src/kernels/sign.cpp:26-33 (f32, i64; NaN kept) */
    NERT_UN_ERF,        /* src/kernels/erf.cpp:48 */
    NERT_UN_ELU,        /* src/kernels/elu.cpp:62-66, p0 = alpha */
    NERT_UN_CLIP,       /* src/kernels/clip.cpp:49-75, p0 = lo, p1 = hi (f32) */
    NERT_UN_ISNAN,      /* src/kernels/is_nan.cpp, f32 -> bool */
    NERT_UN_NOT         /* src/kernels/not.cpp, bool -> bool */
};

/* y[i] = op(x[i]) over `count` elements of `dtype` (F32 or I64). */
int nert_hip_unary(int op, int dtype, const void* x, void* y, int64_t count, double p0, double p1, void* stream);
/* int64 Clip with exact 64-bit bounds (src/kernels/clip.cpp:92-95). */
int nert_hip_clip_i64(const int64_t* x, int64_t* y, int64_t count, int64_t lo, int64_t hi, void* stream);

enum nert_binary_op {
    NERT_BIN_ADD = 0,      /* src/kernels/add.cpp:96-131 (f32, i64) */
    NERT_BIN_SUB,          /* src/kernels/sub.cpp */
    NERT_BIN_MUL,          /* src/kernels/mul.cpp */
    NERT_BIN_DIV,          /* src/kernels/div.cpp (i64 truncates; zero divisor sets flag bit 0) */
    NERT_BIN_POW,          /* src/kernels/pow.cpp (f32; exponent 2 is x*x) */
    NERT_BIN_MOD,          /* src/kernels/mod.cpp (i64 truncating remainder) */
    NERT_BIN_MAX,          /* src/kernels/max.cpp (std::max NaN order) */
    NERT_BIN_MIN,          /* src/kernels/min.cpp */
    NERT_BIN_EQUAL,        /* -> bool, src/kernels/equal.cpp */
    NERT_BIN_GREATER,
    NERT_BIN_LESS,
    NERT_BIN_GREATER_EQUAL,
    NERT_BIN_LESS_EQUAL,
    NERT_BIN_AND,          /* bool x bool -> bool */
    NERT_BIN_OR,
    NERT_BIN_WHERE         /* three operands: bool cond, x, y (f32 or i64) */
};

/* NumPy multidirectional broadcast of 2 (or 3 for WHERE) operands into
 * `out` of rank out_rank and dims out_dims. Operand k has input_ranks[k]
 * dims input_dims[k], right-aligned against out_dims. `dtype` is the
 * operands' element type (for WHERE, of operands 1 and 2). Shared form of the
 * reference's AlignedStrides walk (src/kernels/add.cpp:55-93). */
int nert_hip_broadcast(int op, int dtype, int n_inputs, const void* const* inputs, const int64_t* const* input_dims,
                       const int* input_ranks, void* out, int out_rank, const int64_t* out_dims, void* stream);

/* Element conversion (src/kernels/cast.cpp). to_int32 = 1 emulates ONNX
 * INT32 on int64 lanes (saturating, NaN -> 0). */
int nert_hip_cast(int src_dtype, int dst_dtype, int to_int32, const void* x, void* y, int64_t count, void* stream);
/* Fills `count` elements: F32 takes fvalue, I64 and BOOL take ivalue. */
int nert_hip_fill(int dtype, void* y, int64_t count, double fvalue, int64_t ivalue, void* stream);

/* ---------------------------------------------------------------- pools --- */

typedef struct nert_pool_desc {
    int64_t batch, channels;
    int64_t in[2], out[2], kernel[2], stride[2], dilation[2];
    int64_t pad_begin[2], pad_end[2];
    int64_t count_include_pad; /* AveragePool only */
} nert_pool_desc;

/* src/kernels/max_pool.cpp:138-239 (primary output). */
int nert_hip_maxpool2d_f32(const float* x, float* y, const nert_pool_desc* d, void* stream);
/* src/kernels/average_pool.cpp. */
int nert_hip_avgpool2d_f32(const float* x, float* y, const nert_pool_desc* d, void* stream);
/* Mean of each of `planes` contiguous runs of `spatial` elements;
 * src/kernels/global_average_pool.cpp:32-69. */
int nert_hip_global_avgpool_f32(const float* x, float* y, int64_t planes, int64_t spatial, void* stream);

/* ----------------------------------------------------------- reductions --- */

enum nert_reduce_op {
    NERT_RED_SUM = 0, /* src/kernels/reduce_sum.cpp (f32 in double, i64 exact) */
    NERT_RED_MEAN,    /* src/kernels/reduce_mean.cpp */
    NERT_RED_MAX,     /* src/kernels/reduce_max.cpp (std::max from lowest()) */
    NERT_RED_L2       /* src/kernels/reduce_l2.cpp */
};

/* Reduces the axes flagged in `reduced` (one byte per axis of `dims`); the
 * output holds the kept axes in order (keepdims does not change the data). */
int nert_hip_reduce(int op, int dtype, const void* x, void* y, int rank, const int64_t* dims, const uint8_t* reduced,
                    void* stream);
/* Softmax over `dim` with x viewed as [outer, dim, inner]
 * (src/kernels/softmax.cpp:47-120). */
int nert_hip_softmax_f32(const float* x, float* y, int64_t outer, int64_t dim, int64_t inner, void* stream);
/* LayerNormalization over rows of `inner` elements; Scale/B per element or
 * scalar; Mean/InvStdDev outputs optional (NULL)
 * (src/kernels/layer_normalization.cpp:77-160). */
int nert_hip_layernorm_f32(const float* x, const float* scale, int scale_scalar, const float* bias, int bias_scalar,
                           float* y, float* mean_out, float* invstd_out, int64_t rows, int64_t inner, double epsilon,
                           void* stream);
/* sum = a + b (float32, rounded as the Add row rounds), then y =
 * LayerNorm(sum) over rows of `inner` elements with per-element Scale and
 * optional per-element B, bit-identical to running the Add and
 * LayerNormalization rows one after the other, in one pass over a and b. No
 * counterpart in the reference: it backs the runner's FusedAddLayerNorm row
 * (a residual Add feeding a LayerNormalization, as in every pre-LN
 * transformer block). */
int nert_hip_add_layernorm_f32(const float* a, const float* b, const float* scale, const float* bias, float* sum,
                               float* y, int64_t rows, int64_t inner, double epsilon, void* stream);
/* Scaled-dot-product attention, per (batch b, head h):
 *   O = Softmax(scale * Q K^T, last axis) V,
 * Q/K/V element (b, token t, head h, dim d) at q/k/v + b*in_strides[0] +
 * t*in_strides[1] + h*in_strides[2] + d (one stride set for all three: a
 * packed QKV projection output), O's at out + b*out_strides[0] +
 * t*out_strides[1] + h*out_strides[2] + d. head_dim must be 64; Q, K and
 * out 16-byte aligned with strides that are multiples of 4; the token stride
 * at least head_dim and one (batch, head) slice under 2^32 bytes. The same
 * values as the reference's MatMul(Q, K^T), Mul(scale), Softmax and
 * MatMul(P, V) rows (src/kernels/mat_mul.cpp, mul.cpp, softmax.cpp) within
 * the fp32 parity bar; no counterpart of its own in the reference: it backs
 * the runner's FusedAttention row. */
int nert_hip_attention_f32(const float* q, const float* k, const float* v, float* out, int64_t batch, int64_t heads,
                           int64_t seq, int64_t head_dim, const int64_t* in_strides, const int64_t* out_strides,
                           float scale, void* stream);
/* InstanceNormalization over each (n, c) plane
 * (src/kernels/instance_normalization.cpp:44-106). */
int nert_hip_instancenorm_f32(const float* x, const float* scale, const float* bias, float* y, int64_t batch,
                              int64_t channels, int64_t spatial, double epsilon, void* stream);
/* ArgMax along `dim` of [outer, dim, inner] -> int64 [outer, inner]
 * (src/kernels/arg_max.cpp:41-123). */
int nert_hip_argmax(int dtype, const void* x, int64_t* y, int64_t outer, int64_t dim, int64_t inner, int select_last,
                    void* stream);
/* CumSum along `dim` (src/kernels/cum_sum.cpp:40-145). */
int nert_hip_cumsum(int dtype, const void* x, void* y, int64_t outer, int64_t dim, int64_t inner, int exclusive,
                    int reverse, void* stream);

/* ---- Data movement --------------------------------------------------------
 * Copies the box `dims` element by element: destination element c sits at
 * dst + sum_d c_d * dst_strides[d], its source at src + sum_d s_d *
 * src_strides[d] with s_d = c_d, or c_d % src_mods[d] when src_mods is
 * non-NULL and src_mods[d] > 0. Strides count elements of `elem_size` bytes
 * (1, 4 or 8) and may be zero (broadcast) or negative (reversed walk).
 * Serves Transpose, Concat, Split, Slice, Expand and Tile
 * (src/kernels/{transpose,concat,split,slice,expand,tile}.cpp). */
int nert_hip_copy_strided(int elem_size, const void* src, void* dst, int rank, const int64_t* dims,
                          const int64_t* src_strides, const int64_t* dst_strides, const int64_t* src_mods,
                          void* stream);

/* Concatenates n_inputs (1..8) inputs along one axis in one launch: the
 * output is `outer` rows of sum_i row_bytes[i] bytes, row r holding input
 * i's row r (row_bytes[i] bytes at srcs[i] + r * row_bytes[i]) in input
 * order. Inputs with row_bytes 0 may be NULL. Serves Concat
 * (src/kernels/concat.cpp), one launch instead of one copy per input. */
int nert_hip_concat_rows(int n_inputs, const void* const* srcs, const int64_t* row_bytes, void* dst, int64_t outer,
                         void* stream);
/* Pad of a dense tensor: out[c] = in[map(c - begins)] per axis, mode 0
 * constant (fill `fvalue` for float32, `ivalue` for int64), 1 reflect, 2 edge
 * (src/kernels/pad.cpp:43-96). */
int nert_hip_pad(int dtype, const void* x, void* y, int rank, const int64_t* in_dims, const int64_t* out_dims,
                 const int64_t* begins, int mode, double fvalue, int64_t ivalue, void* stream);

/* ---- Index rows --------------------------------------------------------------
 * Gather over x viewed as [outer, dim, inner] with `index_count` int64
 * indices (negative wrap); y is [outer, index_count, inner]. An index still
 * out of range raises error bit 1 (src/kernels/gather.cpp:29-46). */
int nert_hip_gather(int elem_size, const void* x, const int64_t* indices, void* y, int64_t outer, int64_t dim,
                    int64_t index_count, int64_t inner, void* stream);
/* GatherElements: y has the indices' shape `idx_dims`; off-axis coordinates
 * must already lie inside `in_dims` (the row checks the shapes); an index out
 * of range along `axis` raises error bit 1 (src/kernels/gather_elements.cpp:28-71). */
int nert_hip_gather_elements(int elem_size, const void* x, const int64_t* indices, void* y, int rank,
                             const int64_t* in_dims, const int64_t* idx_dims, int axis, void* stream);
/* ScatterND: out = data, then slice s of `updates` lands at the k-tuple
 * indices[s]; duplicates resolve to the last slice, as in the reference's
 * in-order loop. Out-of-range tuples raise error bit 1
 * (src/kernels/scatter_nd.cpp:31-118). */
int nert_hip_scatter_nd(int elem_size, const void* data, const int64_t* indices, const void* updates, void* out,
                        int data_rank, const int64_t* data_dims, int64_t slice_count, int k, void* stream);
/* TopK (largest, sorted) along `dim` of x viewed as [outer, dim, inner]:
 * values [outer, k, inner] f32 and int64 indices, ordered by value
 * descending and equal values by ascending index, -0.0 equal to +0.0
 * (src/kernels/top_k.cpp:125-141). Requires 0 < k <= dim < 2^32. */
int nert_hip_topk_f32(const float* x, float* values, int64_t* indices, int64_t outer, int64_t dim, int64_t inner,
                      int64_t k, void* stream);

/* nert_hip_topk_f32 without any allocation. No counterpart in the reference:
 * it is for callers that cannot allocate device memory -- work being
 * captured into a HIP graph, tight serving loops, harnesses that forbid
 * hipMalloc. Same arguments, results and errors as nert_hip_topk_f32, but
 * the long-row counters, select state and candidates live in a fixed 4 MiB
 * device array that the library holds on each GPU until the process ends
 * (set up by nert_hip_init, which must have run). Rows longer than 4096
 * need about 16 * rows * k + 3 KiB * rows bytes of it; larger requests fail
 * with an error and launch nothing. Every call on one GPU shares that GPU's
 * array, so calls that overlap in time on one GPU (two streams, two
 * threads) race: serialise them. The array keeps the last call's contents;
 * its per-row counters are zeroed once at set-up and every call leaves them
 * zero, and each call clears the rest of what it needs with a kernel (no
 * memset node). */
int nert_hip_topk_f32_noalloc(const float* x, float* values, int64_t* indices, int64_t outer, int64_t dim,
                              int64_t inner, int64_t k, void* stream);
/* Range: y[i] = start + i * delta, float32 rounded after the product and
 * after the sum (src/kernels/range.cpp:62-64), or int64. */
int nert_hip_range(int dtype, double fstart, double fdelta, int64_t istart, int64_t idelta, void* y, int64_t count,
                   void* stream);
/* Writes `count` (<= 16) int64 values passed by value, with no host buffer
 * (capture-safe): the payload of Shape (src/kernels/shape.cpp:66-70). */
int nert_hip_store_i64(int64_t* y, const int64_t* values, int count, void* stream);
/* EyeLike: ones where col - row == k (src/kernels/eye_like.cpp:54-79). */
int nert_hip_eye_like(int dtype, void* y, int64_t rows, int64_t cols, int64_t k, void* stream);

/* ---- Resampling ------------------------------------------------------------ */

enum nert_resize_code {
    /* coordinate_transformation_mode */
    NERT_RESIZE_HALF_PIXEL = 0,
    NERT_RESIZE_PYTORCH_HALF_PIXEL = 1,
    NERT_RESIZE_ALIGN_CORNERS = 2,
    NERT_RESIZE_ASYMMETRIC = 3,
    /* nearest_mode */
    NERT_RESIZE_ROUND_PREFER_FLOOR = 0,
    NERT_RESIZE_ROUND_PREFER_CEIL = 1,
    NERT_RESIZE_FLOOR = 2,
    NERT_RESIZE_CEIL = 3
};
/* Resize of a dense rank <= 8 tensor; scales[d] is the per-axis scale the
 * coordinate transform divides by (src/kernels/resize.cpp:48-123,230-255).
 * linear = 0: nearest (float32 or int64); 1: linear (float32). */
int nert_hip_resize(int dtype, const void* x, void* y, int rank, const int64_t* in_dims, const int64_t* out_dims,
                    const double* scales, int linear, int transform, int nearest, void* stream);

enum nert_grid_padding { NERT_GRID_ZEROS = 0, NERT_GRID_BORDER = 1, NERT_GRID_REFLECTION = 2 };
/* GridSample: X [n,c,h,w], grid [n,ho,wo,2] (x, y in [-1, 1]) -> [n,c,ho,wo]
 * (src/kernels/grid_sample.cpp:41-71,132-157). nearest = 0: bilinear. */
int nert_hip_grid_sample_f32(const float* x, const float* grid, float* y, int64_t n, int64_t c, int64_t h, int64_t w,
                             int64_t ho, int64_t wo, int nearest, int padding, int align_corners, void* stream);

/* ---- Contractions ------------------------------------------------------------
 * Einsum over one (b = NULL) or two float32 operands, resolved by the caller
 * into labels: y is dense over the output labels (out_size, row-major); each
 * element sums, in double, the product of the operands over the summed labels
 * (sum_size, odometer order, last fastest). Strides are per label and operand,
 * in elements; a repeated label (diagonal) carries the sum of its strides
 * (src/kernels/einsum.cpp:205-258). At most 16 labels of each kind.
 * Two-operand equations that are batched matrix products (batch labels, then
 * row labels of a, then column labels of b -- or columns before rows -- each
 * group mergeable into one strided index, every summed label in both
 * operands, at most four batch groups) run on the MFMA GEMM engine with fp32
 * accumulation instead (within 1e-4 of the double sums); the environment
 * variable NERT_HIP_EINSUM_EXACT=1 keeps every equation on the double path. */
int nert_hip_einsum_f32(const float* a, const float* b, float* y, int n_out, const int64_t* out_size,
                        const int64_t* out_stride_a, const int64_t* out_stride_b, int n_sum, const int64_t* sum_size,
                        const int64_t* sum_stride_a, const int64_t* sum_stride_b, void* stream);
/* 2-D ConvTranspose, NCHW, weight [C, M/group, kh, kw], optional bias [M].
 * geom = {batch, C, M, group, in_h, in_w, out_h, out_w, kh, kw, stride_h,
 * stride_w, pad_top, pad_left, dilation_h, dilation_w}; strides > 0
 * (src/kernels/conv_transpose.cpp:76-188). */
int nert_hip_conv_transpose_f32(const float* x, const float* w, const float* bias, float* y, const int64_t* geom,
                                void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NERT_HIP_H */
