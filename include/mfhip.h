/*
 * mfhip.h -- C ABI of libmfhip.so, the MI355X (gfx950) transformer
 * evaluation backend for MetalFish.
 *
 * This is the drop-in boundary below MetalFish's `NN::Network` interface
 * (reference src/nn/network.h:38-51).  A C++ adapter (metalfish_amd/csrc/
 * host/hip_network.{h,cpp}, class HipNetwork) implements NN::Network on top
 * of these calls; Python binds them with ctypes (metalfish_amd/backend.py).
 * Plain pointers and sizes only; no exceptions cross this boundary.  Every
 * call returns MFH_OK or a negative status and leaves a message for
 * mfh_last_error() (thread-local).
 *
 * Format enums take the values of the reference's NetworkFormat proto
 * (reference src/nn/proto/net.proto:278-342) so an adapter can pass a loaded
 * weights file's format fields through unchanged.
 */
#ifndef MFHIP_H
#define MFHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  MFH_OK = 0,
  MFH_ERR_INVALID = -1,     /* bad argument, shape or missing tensor */
  MFH_ERR_HIP = -2,         /* HIP runtime error */
  MFH_ERR_UNSUPPORTED = -3, /* net structure outside what the kernels handle */
  MFH_ERR_NO_DEVICE = -4,   /* no usable gfx950 device */
  MFH_ERR_OUT_OF_MEMORY = -5
};

/* NetworkFormat.NetworkStructure (net.proto:278-287). */
enum { MFH_NETWORK_ATTENTIONBODY_WITH_HEADFORMAT = 6,
       MFH_NETWORK_ATTENTIONBODY_WITH_MULTIHEADFORMAT = 7 };
/* NetworkFormat.PolicyFormat / ValueFormat (net.proto:293-305). */
enum { MFH_POLICY_ATTENTION = 3 };
enum { MFH_VALUE_CLASSICAL = 1, MFH_VALUE_WDL = 2 };
/* NetworkFormat.InputEmbeddingFormat (net.proto:340-342). */
enum { MFH_INPUT_EMBEDDING_PE_MAP = 1, MFH_INPUT_EMBEDDING_PE_DENSE = 2 };
/* NetworkFormat.ActivationFunction (net.proto:317-326). */
enum {
  MFH_ACTIVATION_DEFAULT = 0,
  MFH_ACTIVATION_MISH = 1,
  MFH_ACTIVATION_RELU = 2,
  MFH_ACTIVATION_NONE = 3,
  MFH_ACTIVATION_TANH = 4,
  MFH_ACTIVATION_SIGMOID = 5,
  MFH_ACTIVATION_SELU = 6,
  MFH_ACTIVATION_SWISH = 7,
  MFH_ACTIVATION_RELU_2 = 8
};
/* NetworkFormat.MovesLeftFormat (net.proto:310-313). */
enum { MFH_MOVES_LEFT_NONE = 0, MFH_MOVES_LEFT_V1 = 1 };
/* NetworkFormat.DefaultActivation (net.proto:331-332). */
enum { MFH_DEFAULT_ACTIVATION_RELU = 0, MFH_DEFAULT_ACTIVATION_MISH = 1 };
/* Storage of the GEMM weights on the device.  BF16: each weight rounded to
 * bf16.  FP8: each output row of a GEMM weight stored as OCP e4m3 codes
 * (round to nearest even, saturating at 448) with one fp32 scale
 * max|row| / 448; the kernels convert the codes exactly to bf16 and apply the
 * scale to the accumulated row, halving weight bytes. */
enum { MFH_WEIGHTS_BF16 = 0, MFH_WEIGHTS_FP8 = 1 };
/* Activation precision.  BF16: every MFMA operand is one bf16 value (fastest).
 * BF16X2: activations are carried as a bf16 pair hi + lo (lo = bf16(x - hi))
 * and every product takes two (GEMMs) or three (attention, policy map)
 * bf16 MFMAs, giving ~16-bit activation precision against the exact bf16
 * weights at twice the MFMA work.  BF16X2_GEMM: the pair only for the inputs
 * of the dense layers and the policy map; attention Q/K/V, its
 * probabilities, the smolgen activations and bias stay single bf16.
 * FP8 (needs MFH_WEIGHTS_FP8): from 2048 token rows (32 positions) up, the
 * Q|K|V, out-projection and FFN GEMMs of the encoder layers run on the fp8
 * MFMA, their inputs quantised per row to OCP e4m3 (scale max|row| / 448)
 * just before each GEMM; everything else as in BF16.
 * FP8 is EXPERIMENTAL and does not meet the parity gates against the fp32
 * CPU backend: on the random-init BT4-shape net, same top-1 move on ~80 % of
 * positions, policy max-abs ~0.15, WDL ~1e-2 (the gates are 99.5 %, 2e-2
 * and 5e-3).  mfh_net_create refuses it (MFH_ERR_UNSUPPORTED) unless the
 * environment sets METALFISH_HIP_EXPERIMENTAL_FP8=1.  For e4m3 weights
 * within the gates use MFH_WEIGHTS_FP8 with BF16X2. */
/* BF16X2_FP8LO: BF16X2 with the lo parts of the encoder layers' dense-layer
 * inputs (Q|K|V, out-projection, FFN1, FFN2) carried as OCP e4m3 codes of
 * lo * 2^10, from 8192 token rows (128 positions) up: each of those GEMMs
 * is hi . W on the bf16 MFMA plus lo . W8 on the fp8 MFMA
 * (v_mfma_f32_16x16x128_f8f6f4), W8 the e4m3 codes of each weight row over a
 * power-of-two (bf16 weights) or its max|row| / 448 (fp8 weights) scale.
 * The lo product carries ~4 of lo's 8 bits; the product is ~2^-13 relative
 * instead of BF16X2's 2^-17, at three quarters of BF16X2's MFMA time.
 * Attention reads the lo parts of Q, K and V as the same e4m3 codes (its
 * MFMAs stay bf16) and the smolgen bias as bf16 + e4m3 codes of its lo
 * part; the residual stream and the heads are as in BF16X2.  Below 8192
 * rows the whole forward is BF16X2.  The embedding and FFN widths must be
 * multiples of 128 (mfh_net_create returns MFH_ERR_UNSUPPORTED otherwise). */
enum {
  MFH_PRECISION_BF16 = 0,
  MFH_PRECISION_BF16X2 = 1,
  MFH_PRECISION_BF16X2_GEMM = 2,
  MFH_PRECISION_FP8 = 3,
  MFH_PRECISION_BF16X2_FP8LO = 4
};

/* Network description: the format fields of the weights file plus the
 * attention head count (Weights.headcount) and run-time sizing. */
typedef struct {
  int network;            /* MFH_NETWORK_ATTENTIONBODY_* */
  int policy;             /* MFH_POLICY_ATTENTION */
  int value;              /* MFH_VALUE_WDL or MFH_VALUE_CLASSICAL */
  int moves_left;         /* 0, or 1 (MOVES_LEFT_V1) for a moves-left head */
  int input_embedding;    /* MFH_INPUT_EMBEDDING_PE_DENSE or _PE_MAP */
  int default_activation; /* MFH_DEFAULT_ACTIVATION_* */
  int ffn_activation;     /* MFH_ACTIVATION_*; DEFAULT follows default_activation */
  int smolgen_activation; /* MFH_ACTIVATION_*; DEFAULT follows default_activation */
  int headcount;          /* body attention heads; head depth must be 32 */
  int weights_dtype;      /* MFH_WEIGHTS_BF16 or MFH_WEIGHTS_FP8 */
  int precision;          /* MFH_PRECISION_* */
  int max_batch;          /* largest batch one eval call accepts (>= 1) */
  int device;             /* HIP device ordinal, -1 = current device */
  int pol_headcount;      /* policy encoder heads (Weights.pol_headcount); 0 without
                             policy encoder layers */
  int fused_layernorm;    /* residual GEMM + the LayerNorm after it as one
                             row-panel launch (batches >= 128, BF16X2 and
                             BF16X2_GEMM): 1 always; 0 chooses as measured on
                             MI355X: on with fp8 weights, off with bf16 weights
                             (tiled GEMM, then the LayerNorm kernel) */
} mfh_net_desc;

/* One weight tensor, named as in the reference's weight inventory
 * (e.g. "body.ip_emb_w", "body.encoder.3.mha.q_w", "policy.vanilla.ip4_pol_w",
 * "value.winner.ip1_val_w"); matrices are row-major [out][in]. */
typedef struct {
  const char *name;
  const float *data; /* host fp32 */
  uint64_t count;    /* number of floats */
} mfh_tensor;

typedef struct mfh_net mfh_net;

/* Shape inference, weight packing and upload, workspace allocation for
 * desc->max_batch positions.  Replaces the backend constructor
 * (reference src/nn/cuda/cuda_network.cpp:235-321) and its call from
 * NN::CreateNetwork (reference src/nn/network.cpp:137-208). */
int mfh_net_create(const mfh_net_desc *desc, const mfh_tensor *tensors,
                   int n_tensors, mfh_net **out);

void mfh_net_destroy(mfh_net *net);

/* Forward pass on host buffers in the reference's packed input contract
 * (reference src/nn/input_plane_packing.h:61-83): masks[batch*112] and
 * values[batch*112].  Outputs: policy[batch*1858] raw logits in the 1858
 * order, wdl[batch*3] (WDL nets) or value[batch] (classical value head),
 * moves_left[batch] (nets with a moves-left head; NULL to skip; must be NULL
 * otherwise).  Inputs are staged through pinned buffers with
 * asynchronous copies on the net's stream; the call returns when outputs are
 * in place.  Calls on one net are serialised (reference
 * src/nn/cuda/cuda_network.cpp:442).  batch must be 1..max_batch. */
int mfh_net_eval(mfh_net *net, int batch, const uint64_t *masks,
                 const float *values, float *policy, float *wdl,
                 float *moves_left);

/* Same, from unpacked planes[batch*112*64] (NN::InputPlanes layout,
 * reference src/nn/input_planes.h:22-29); packing happens straight into the
 * pinned staging buffer. */
int mfh_net_eval_planes(mfh_net *net, int batch, const float *planes,
                        float *policy, float *wdl, float *moves_left);

/* Forward pass on device-resident buffers (no host copies, no
 * synchronisation), enqueued on `stream` (a hipStream_t; NULL is the
 * default stream).  Outputs are ready when that stream reaches this point.
 * All calls on one net share its workspace, so each call's device work is
 * ordered after the previous call's, whatever stream either ran on (the
 * new stream waits on an event the previous call recorded); calls on
 * different streams therefore run one after another on the device. */
int mfh_net_eval_device(mfh_net *net, int batch, const uint64_t *d_masks,
                        const float *d_values, float *d_policy, float *d_wdl,
                        void *stream);

/* Forward pass plus the MCTS priors of each position's legal moves, so that
 * only the priors and the value head output cross PCIe (about 35 floats per
 * position instead of 1858).  Replaces the host-side gather of
 * NNMCTSEvaluator::BuildResult (reference src/mcts/evaluator.cpp:181-224)
 * and the softmax of ApplyNNPolicyToNode (reference src/mcts/search.cpp:
 * 127-199), which keep working unchanged on mfh_net_eval's logits.
 *
 * The moves of position b are move_indices[move_offsets[b] ..
 * move_offsets[b + 1]) in the caller's edge order: policy indices as
 * MoveToNNIndex gives them (side-to-move mirroring and transform applied by
 * the caller); an index outside 0..1857 reads logit 0, as BuildResult does.
 * move_offsets[0] must be 0 and each position has 0..256 moves (kMaxEdges,
 * search.cpp:49).  priors[move_offsets[batch]] receives, per position,
 * exp((logit - max) / softmax_temp) with the reference's Schraudolph
 * exponential (src/mcts/core.h:38-44), divided by their sequential sum (1/n
 * each when the sum is not positive): the same float operations in the same
 * order as the reference, so the priors equal the CPU computation on the
 * same logits bit for bit.  wdl and moves_left as in mfh_net_eval. */
int mfh_net_eval_priors(mfh_net *net, int batch, const uint64_t *masks,
                        const float *values, const int32_t *move_offsets,
                        const int16_t *move_indices, float softmax_temp,
                        float *priors, float *wdl, float *moves_left);

/* Same on device-resident buffers, enqueued on `stream` like
 * mfh_net_eval_device; d_policy receives the raw logits on the way.  The
 * offsets are read on the device and are not checked: the caller keeps them
 * within the rules above. */
int mfh_net_eval_priors_device(mfh_net *net, int batch, const uint64_t *d_masks,
                               const float *d_values, const int32_t *d_move_offsets,
                               const int16_t *d_move_indices, float softmax_temp,
                               float *d_policy, float *d_priors, float *d_wdl,
                               void *stream);

/* mfh_net_eval_device for a net with a moves-left head, which also writes
 * d_moves_left[batch] (the reference's NetworkOutput::moves_left,
 * network_output_decoder.cpp:68-71).  mfh_net_eval_device leaves the
 * moves-left output in the net's workspace. */
int mfh_net_eval_device_moves_left(mfh_net *net, int batch,
                                   const uint64_t *d_masks, const float *d_values,
                                   float *d_policy, float *d_wdl,
                                   float *d_moves_left, void *stream);

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  mfh_net_eval_device without the net's workspace: the
 * forward's activations, split-K partials and smolgen bias live in the
 * library's static 64 MiB device array (one copy per device, held until the
 * process ends), and the call allocates nothing (no hipMalloc, no graph, no
 * profiler events; the kernels run eagerly on `stream`).  batch must be 1 up
 * to the largest batch below 32 whose workspace fits that array (mfh_net_info
 * reports it; for the BT4 shape 15 in BF16X2, 19 in BF16X2_GEMM, 27 in BF16,
 * and 31 for the 256-wide config-1 net); a larger batch is rejected with
 * MFH_ERR_INVALID.  Outputs equal
 * mfh_net_eval_device's bit for bit.  Every call on a device, from any net,
 * shares that device's array, which keeps the last call's contents: calls
 * that overlap on one device (different streams, or threads of different
 * nets) race, so the caller orders them.  Calls on one net are serialised on
 * the host like the other entry points. */
int mfh_net_eval_device_noalloc(mfh_net *net, int batch,
                                const uint64_t *d_masks, const float *d_values,
                                float *d_policy, float *d_wdl, void *stream);

/* Human-readable description (GetNetworkInfo, reference network.h:47). */
int mfh_net_info(const mfh_net *net, char *buf, size_t len);

/* Capabilities (BackendCapabilities, reference network.h:21-36). */
typedef struct {
  int has_wdl;
  int has_moves_left;
  int max_batch_size;
  int device;
  char device_name[64];
  char arch_name[32];
  uint64_t weight_bytes;
  uint64_t workspace_bytes;
} mfh_capabilities;
int mfh_net_capabilities(const mfh_net *net, mfh_capabilities *out);

/* Graph execution (the counterpart of BackendConfig::cuda_graph_execution,
 * reference src/nn/network.h:58 and cuda_network.cpp:312): when enabled (the
 * default), the forward for a batch size and set of device buffers runs
 * eagerly once and is then captured into a HIP graph that later calls
 * replay with a single launch.  A net caches up to 64 graphs (one per batch
 * size and buffer set of mfh_net_eval_device; mfh_net_eval's pinned buffers
 * are one set); keys seen after the cache is full run eagerly, without a
 * capture, and the cached graphs stay.  Profiling bypasses graphs.
 * Changing the setting drops the cached graphs. */
int mfh_net_set_graphs(mfh_net *net, int enabled);

/* Stage profiler (the counterpart of the reference's METALFISH_CUDA_PROFILE
 * stage timers, reference src/nn/cuda/cuda_stage_executor.cpp:421-482):
 * while enabled, every kernel launch of an eval call is bracketed by HIP
 * events recorded on the stream it is launched on.  mfh_net_profile
 * synchronises and returns, per kernel kind, the launch count, summed
 * duration and the algorithmic work of those launches (GEMM/attention
 * FLOPs = 2*M*N*K of the useful products, bytes = minimal HBM traffic). */
typedef struct {
  char name[48];
  int launches;
  double milliseconds;
  double flops;
  double bytes;
} mfh_profile_entry;
int mfh_net_set_profiling(mfh_net *net, int enabled);
int mfh_net_profile(mfh_net *net, mfh_profile_entry *out, int capacity,
                    int *count);
int mfh_net_profile_reset(mfh_net *net);

/* PackInputPlanesRaw (reference src/nn/input_plane_packing.h:61-83):
 * planes[batch*112*64] -> masks[batch*112], values[batch*112]. */
int mfh_pack_planes(int batch, const float *planes, uint64_t *masks,
                    float *values);

/* The FP8 weight quantisation of MFH_WEIGHTS_FP8 on the host (no device
 * needed; no counterpart in the reference, which stores fp16/fp32 weights):
 * w[rows*cols] row-major -> codes[rows*cols] e4m3 and scale[rows]. */
int mfh_debug_quantize_fp8(int rows, int cols, const float *w, uint8_t *codes,
                           float *scale);

/* ---- Network files (no device needed) ----------------------------------
 *
 * A reader for the reference's `.pb` / `.pb.gz` network files
 * (reference src/nn/proto/net.proto) that needs no libprotobuf.  Loading
 * applies the reference's legacy format fix-ups and layer decoding
 * (LINEAR16 / FLOAT16 / BFLOAT16 / FLOAT32), folds convolution batch norms,
 * resolves the selected policy and value heads ("vanilla", "winner") and
 * yields the weight inventory: the tensors mfh_net_create takes, under the
 * same names. */
typedef struct mfh_weights mfh_weights;

/* NetworkFormat fields after the fix-ups (values as in net.proto:253-343;
 * input_embedding is PE_MAP when the file leaves it unset, as
 * DescribeNetworkFormat reads it, reference src/nn/network_format.cpp:97-100)
 * and the head counts. */
typedef struct {
  int input;
  int output;
  int network;
  int policy;
  int value;
  int moves_left;
  int default_activation;
  int smolgen_activation;
  int ffn_activation;
  int input_embedding;
  int headcount;     /* Weights.headcount */
  int pol_headcount; /* pol_headcount of the selected policy head */
} mfh_weights_format;

/* LoadWeights (reference src/nn/loader.cpp:162-189: names ending in ".gz"
 * are gzip-decompressed, the magic must be 0x1c0, FixOlderWeightsFile
 * 86-135 is applied) followed by MultiHeadWeights (src/nn/weights.cpp:
 * 216-291) and CreateNetworkWeightInventory for the selected heads
 * (src/nn/network_weight_inventory.cpp:332-352).  Errors (MFH_ERR_INVALID)
 * carry the reference's messages, e.g. "Invalid weight file: bad magic
 * number", "RPE weights file not supported.". */
int mfh_weights_load(const char *path, mfh_weights **out);

/* The same on an in-memory serialised Net message (ParseWeightsProto,
 * reference src/nn/loader.cpp:137-158; not gzip). */
int mfh_weights_parse(const void *data, uint64_t bytes, mfh_weights **out);

/* Format fields and head counts.  With desc non-NULL, also fills the format
 * fields, headcount and pol_headcount of a net description, as DescribeNetworkFormat reads
 * them (reference src/nn/network_format.cpp:72-127), leaving weights_dtype,
 * precision, max_batch and device as the caller set them.  Either pointer
 * may be NULL. */
int mfh_weights_describe(const mfh_weights *w, mfh_weights_format *format,
                         mfh_net_desc *desc);

/* The inventory (NetworkWeightInventory::tensors, reference
 * src/nn/network_weight_inventory.h:33-56): names, fp32 data and element
 * counts, in inventory order.  Valid until mfh_weights_free. */
int mfh_weights_tensors(const mfh_weights *w, const mfh_tensor **tensors,
                        int *count);

/* Dims of tensor `index` (the layer's dims, or its flat size when the file
 * gives none; NetworkWeightTensorView::dims). */
int mfh_weights_tensor_dims(const mfh_weights *w, int index,
                            const uint32_t **dims, int *ndims);

void mfh_weights_free(mfh_weights *w);

/* Number of visible devices (0 without a GPU). */
int mfh_device_count(int *count);

const char *mfh_last_error(void);

/* ---- Parity hooks (used by the test suite) ---------------------------- */

/* Unpacks packed inputs on the device into planes[batch*112*64] (host). */
int mfh_debug_unpack_planes(int batch, const uint64_t *masks,
                            const float *values, float *planes);

/* C[M,N] = act(A[M,K] . W[N,K]^T + bias) with bf16 operands (host arrays of
 * raw bf16 bits), fp32 output.  act is MFH_ACTIVATION_*. */
int mfh_debug_gemm_bf16(int M, int N, int K, const uint16_t *A,
                        const uint16_t *W, const float *bias, int act,
                        float *C);

/* fp8 x fp8 GEMM (the kernel of the fp8-activation precision) on host
 * arrays, for tests: C[M,N] = act((A8 . W8^T) * ascale[m] * wscale[n] +
 * bias) in fp32, A8 [M,K] and W8 [N,K] OCP e4m3 codes with row scales.
 * K % 128 == 0, M >= 2048.  No counterpart in the reference. */
int mfh_debug_gemm_fp8(int M, int N, int K, const uint8_t *A8, const float *ascale,
                       const uint8_t *W8, const float *wscale, const float *bias,
                       int act, float *C);

/* The GEMM of the BF16X2_FP8LO precision on host arrays, for tests: the hi
 * product on the bf16 MFMA plus the lo product on the fp8 MFMA, accumulated
 * together: acc = A . W^T + A_lo8 . W_lo8^T, A and W [M,K] / [N,K] bf16 bits,
 * A_lo8 and W_lo8 OCP e4m3 codes of the same shapes (code values, no
 * scale), then act(acc * wscale[n] + bias).  Into C (fp32), or as bf16 bits
 * C_hi with the lo part C_lo8 = e4m3((out - C_hi) * 2^10) (the BF16X2_FP8LO
 * activation codes).  K % 128 == 0.  No counterpart in the reference. */
int mfh_debug_gemm_lo8(int M, int N, int K, const uint16_t *A, const uint8_t *A_lo8,
                       const uint16_t *W, const uint8_t *W_lo8, const float *wscale,
                       const float *bias, int act, float *C, uint16_t *C_hi,
                       uint8_t *C_lo8);

/* The device row quantiser of the fp8-activation precision on host arrays,
 * for tests: rows of bf16 bits x (+ lo plane x_lo) as OCP e4m3 codes with
 * scale = max|row| / 448 per row, the arithmetic of mfh_debug_quantize_fp8.
 * No counterpart in the reference. */
int mfh_debug_quantize_rows_e4m3(int rows, int cols, const uint16_t *x,
                                 const uint16_t *x_lo, uint8_t *codes,
                                 float *scales);

/* Few-row GEMM (the kernel of the batch-1 encoder layers, reference
 * cpu_network.cpp:822-890 with the LayerNorm of 424-460 applied to its
 * input) on host arrays, for tests.  The activation operand is A [M,K] bf16
 * bits (A_lo: optional lo plane), or, with x set, the LayerNorm of fp32 rows
 * x [ceil(M / rows_per_src), rows_per_src * K]: row r reads segment
 * r % rows_per_src of source row r / rows_per_src, normalised over the whole
 * source row with gamma / beta of that width and eps (ln_split adds the
 * normalised value's bf16 lo plane to the product; y_hi / y_lo / y32, when
 * set with rows_per_src == 1, receive the normalised rows [M,K]).  W [N,K]
 * bf16 bits.  out_mode 0: out = act(A.W^T + bias) as bf16 bits (+ out_lo);
 * 1: fp32 act(A.W^T + bias); 2: fp32 resid + alpha (A.W^T + bias) with
 * resid32 or resid_hi + resid_lo.  stats (fp32 modes, optional): per
 * workgroup part p and row m the sum and sum of squares of the outputs at
 * stats[2 (p M + m)], *parts parts.  No counterpart in the reference. */
int mfh_debug_skinny_gemm(int M, int N, int K, const uint16_t *A,
                          const uint16_t *A_lo, const float *x, int rows_per_src,
                          float eps, const float *gamma, const float *beta,
                          int ln_split, const uint16_t *W, const float *bias,
                          int act, int out_mode, const float *resid32,
                          const uint16_t *resid_hi, const uint16_t *resid_lo,
                          float alpha, void *out, uint16_t *out_lo, float *stats,
                          int *parts, uint16_t *y_hi, uint16_t *y_lo, float *y32);

/* Row-panel GEMM (the kernel behind the batch >= 128 residual + LayerNorm
 * steps, reference cpu_network.cpp:1256-1259 / 1318-1397 then 1399-1457) on
 * host arrays, for tests.  A [M,K] bf16 bits (A_lo: optional split-precision
 * lo plane), weights W [N,K] bf16 bits or W8 e4m3 codes with wscale[N].
 * layernorm = 0: out = act(A.W^T + bias) as bf16 hi (+ lo) planes.
 * layernorm = 1: out = LN(resid + alpha (A.W^T + bias)) with gamma, beta,
 * eps over each row of N, residual fp32 resid32 or the pair resid_hi +
 * resid_lo; bf16 hi (+ lo) planes and optionally fp32 out_f32. */
int mfh_debug_panel_gemm(int M, int N, int K, const uint16_t *A,
                         const uint16_t *A_lo, const uint16_t *W,
                         const uint8_t *W8, const float *wscale,
                         const float *bias, int act, int layernorm,
                         const float *resid32, const uint16_t *resid_hi,
                         const uint16_t *resid_lo, float alpha, float eps,
                         const float *gamma, const float *beta,
                         uint16_t *out_hi, uint16_t *out_lo, float *out_f32);

/* One body encoder layer alone (cpu_network.cpp:1027-1266 and 1318-1457;
 * the isolated encoder-layer microbenchmark): writes x (bf16 bits
 * [batch*64, E]; x_lo its lo plane, required in the split precisions) into
 * the residual stream, runs layer `layer` `iterations` times on the net's
 * stream (each run on the previous run's output) and returns the average
 * milliseconds per run.  With profiling on, mfh_net_profile reports the
 * layer's kernels. */
int mfh_debug_encoder_layer(mfh_net *net, int batch, int layer, int iterations,
                            const uint16_t *x, const uint16_t *x_lo, float *ms);

/* Copies a named workspace tensor left by the last eval call (or
 * mfh_debug_encoder_layer run) to host memory: "body" (fp32 [B*64,E],
 * encoder output; with no encoder layers the input-embedding output),
 * "policy_qk" (bf16 [B*64,2Dp]), the last encoder layer's "act" (bf16
 * [B*64,E], its output), "qkv" (bf16 [B*64,3E]), "ctx" (bf16 [B*64,E],
 * attention output), "hid" (bf16 [B*64,F], FFN hidden rows) and "pre"
 * (fp32 [B*64,E], the FFN residual sum before its LayerNorm); bf16 tensors
 * are the hi plane in split precision.  In the FP8 precision also
 * "act_e4m3" / "ctx_e4m3" / "hid_e4m3" (u8 codes, the FFN1, out-projection
 * and FFN2 inputs) with "act_scale" / "ctx_scale" / "hid_scale" (fp32 per
 * row).  bytes must equal the tensor's size for the last batch. */
int mfh_net_debug_tensor(mfh_net *net, const char *name, void *out,
                         uint64_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* MFHIP_H */
