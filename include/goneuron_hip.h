/*
 * goneuron_hip.h — C ABI of libgoneuron_hip.so, the MI355X (gfx950) training
 * backend for GoNeuron's fp32 training step (forward + backward + Adam).
 *
 * The library replaces the reference's per-sample CPU loop and its Metal cgo
 * bridge.  Every entry point below names the reference interface it stands in
 * for (paths relative to the GoNeuron tree).  Conventions:
 *   - every call returns an int status: GN_OK (0) or a negative GN_ERR_* code;
 *     gn_last_error() gives the message of the last failure on a context
 *     (the reference's Metal ABI returns void and drops errors,
 *     internal/layer/metal.go:270-274);
 *   - host pointers are read or written only during the call, never retained;
 *   - "_device" entry points take device pointers (HBM-resident inputs);
 *   - one HIP stream per context; a context is not thread-safe (the Go side
 *     serialises calls with a mutex, as MetalDevice.mu does, metal.go:70).
 */
#ifndef GONEURON_HIP_H
#define GONEURON_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define GN_OK 0
#define GN_ERR_INVALID (-1)     /* bad argument (null, size, kind) */
#define GN_ERR_HIP (-2)         /* HIP runtime error */
#define GN_ERR_OOM (-3)         /* device allocation failed */
#define GN_ERR_UNSUPPORTED (-4) /* layer/activation combination not built */
#define GN_ERR_SHAPE (-5)       /* input size mismatch (layer.go:347-349) */
#define GN_ERR_INJECTED (-6)    /* forced by gn_debug_fail_next */
#define GN_ERR_NO_DEVICE (-7)   /* no HIP device */
#define GN_ERR_INDEX (-8)       /* index out of range (embedding.go:126-128) */

/* ---- activation codes ---------------------------------------------------
 * A layer carries the activation *object* the Go code was given and whether it
 * was a pointer (&activations.Softmax{}) or a value (activations.Softmax{}),
 * because Dense dispatches on cacheActivationType (layer.go:183-205), which
 * only recognises pointer Softmax/LogSoftmax: the facade's values run as
 * identity forward and NaN derivative (activations.go:150-158). */
#define GN_ACT_NIL 0
#define GN_ACT_RELU 1
#define GN_ACT_SIGMOID 2
#define GN_ACT_TANH 3
#define GN_ACT_SOFTMAX 4
#define GN_ACT_LOGSOFTMAX 5
#define GN_ACT_LINEAR 6
#define GN_ACT_GELU 7   /* value activations.GELU{}: identity forward, GELU' backward */

/* ---- layer kinds (the []layer.Layer given to goneuron.NewSequential) ----- */
#define GN_LAYER_DENSE 1         /* layer.NewDense            layer.go:267 */
#define GN_LAYER_DROPOUT 2       /* layer.NewDropout          dropout.go:47 */
#define GN_LAYER_CONV2D 3        /* layer.NewConv2D           conv2d.go:74 */
#define GN_LAYER_MAXPOOL2D 4     /* layer.NewMaxPool2D        maxpool2d.go:45 */
#define GN_LAYER_FLATTEN 5       /* layer.NewFlatten          reshape.go:29 */
#define GN_LAYER_EMBEDDING 6     /* layer.NewEmbedding        embedding.go */
#define GN_LAYER_POSENC 7        /* layer.NewPositionalEncoding transformer.go:51 */
#define GN_LAYER_TRANSFORMER 8   /* layer.NewTransformerBlockE transformer.go:908 */
#define GN_LAYER_CLSPOOL 9       /* layer.NewCLSPooling       transformer.go:1679 */
#define GN_LAYER_LSTM_UNROLLER 10 /* SequenceUnroller(LSTM)   unroller.go:57, lstm.go */
#define GN_LAYER_AVGPOOL2D 11    /* layer.NewAvgPool2D        avgpool2d.go:50 */
#define GN_LAYER_RMSNORM 12      /* layer.NewRMSNorm          rmsnorm.go:49 */
#define GN_LAYER_SWIGLU 13       /* layer.NewSwiGLU           swiglu.go:47 */
#define GN_LAYER_BATCHNORM2D 14  /* layer.NewBatchNorm2D      batchnorm2d.go:70 */
#define GN_LAYER_GRU_UNROLLER 15 /* SequenceUnroller(GRU)     unroller.go:57, gru.go:83 */
#define GN_LAYER_MOE 16          /* layer.NewMoE              moe.go:47 */
#define GN_LAYER_MHA 17          /* layer.NewMultiHeadAttentionE transformer.go:283 (dim, num_heads,
                                    seq_len, causal; parameters start at 0, transformer.go:367-379) */
#define GN_LAYER_LAYERNORM 18    /* layer.NewLayerNorm        layernorm.go:57 (dim = normalizedShape,
                                    eps; gamma 1, beta 0) */
#define GN_LAYER_GAP1D 19        /* layer.NewGlobalAveragePooling1D transformer.go:1524 (seq_len, dim) */

/* TransformerBlockExt options (layer.ActivationType, layer.NormType) */
#define GN_BLOCK_ACT_RELU 0
#define GN_BLOCK_ACT_SWIGLU 1
#define GN_BLOCK_ACT_GELU 2
#define GN_BLOCK_NORM_LN 0
#define GN_BLOCK_NORM_RMS 1

#define GN_LOSS_MSE 1            /* loss.MSE          loss.go:38-105 */
#define GN_LOSS_CE 2             /* loss.CrossEntropy loss.go:108-178 */

typedef struct gn_layer_desc {
  int32_t kind;
  int32_t in_size;      /* Dense in / Dropout & Flatten size / first-layer input length */
  int32_t out_size;     /* Dense out / LSTM hidden */
  int32_t act;          /* GN_ACT_* */
  int32_t act_is_ptr;   /* 1 when the Go activation is a pointer */
  int32_t in_channels;  /* Conv2D / MaxPool2D; -1 = lazy (MaxPool runs as 1 channel) */
  int32_t out_channels;
  int32_t kernel, stride, padding;
  float p;              /* Dropout probability */
  int32_t seq_len, num_heads, ff_dim, causal, vocab, dim; /* RMSNorm: dim = normalizedShape */
  int32_t return_sequences;
  float eps;            /* RMSNorm / LayerNorm eps; 0 selects the facade's 1e-5 (goneuron.go:220-236) */
  int32_t block_act;    /* TransformerBlock ff1: GN_BLOCK_ACT_* (transformer.go:199-203) */
  int32_t block_norm;   /* TransformerBlock norms: GN_BLOCK_NORM_* (transformer.go:205-210) */
  int32_t use_rope;     /* TransformerBlock: rotary embeddings on Q and K (transformer.go:212-236) */
  float momentum;       /* BatchNorm2D running-stat momentum, as given (the facade passes 0.1) */
  int32_t no_affine;    /* BatchNorm2D without gamma / beta (NewBatchNorm2D affine = false) */
  int32_t num_experts;  /* MoE experts (<= 64) */
  int32_t top_k;        /* MoE experts per sample */
} gn_layer_desc;

typedef struct gn_adam_desc {   /* opt.NewAdam opt.go:117-126 */
  float lr, beta1, beta2, eps;  /* zeros select the reference defaults */
} gn_adam_desc;

typedef struct gn_info {
  char arch[64];
  int32_t cu_count;
  int64_t hbm_bytes;
  double peak_fp32_mfma_tflops; /* dense fp32 matrix peak */
  double peak_hbm_gbps;
} gn_info;

typedef struct gn_ctx gn_ctx;
typedef struct gn_model gn_model;

/* ---- context -------------------------------------------------------------
 * Replaces layer.GetDefaultDevice / MetalDevice construction
 * (internal/layer/device.go:39-48, metal.go:76-98). */
int gn_available(void);                      /* 1 when a HIP device is present */
int gn_init(int device_ordinal, gn_ctx **out);
void gn_shutdown(gn_ctx *ctx);
const char *gn_last_error(const gn_ctx *ctx);
int gn_device_info(gn_ctx *ctx, gn_info *info);
int gn_sync(gn_ctx *ctx);                    /* waitForMetal, metal_ops.m:1002-1007 */
/* Test hook: the next entry point that takes this context fails with `code`. */
int gn_debug_fail_next(gn_ctx *ctx, int code);

/* ---- device buffers (createMetalBuffer / update / read, metal.go:6-50) --- */
int gn_malloc(gn_ctx *ctx, size_t bytes, void **dptr);
int gn_free(gn_ctx *ctx, void *dptr);
int gn_memcpy_h2d(gn_ctx *ctx, void *dst, const void *src, size_t bytes);
int gn_memcpy_d2h(gn_ctx *ctx, void *dst, const void *src, size_t bytes);
int gn_memset_zero(gn_ctx *ctx, void *dst, size_t bytes);

/* ---- model: Sequential.Compile + Network.initBuffers --------------------
 * sequential.go:26-87, net.go:91-127: layers are built with the reference's
 * seeded LCG initialisation into one device-resident flat arena
 * (params | grads | Adam m | Adam v).  `workers` is the trainBatchParallel
 * worker count W (net.go:588-608; 1 = trainBatchSequential). */
int gn_model_create(gn_ctx *ctx, const gn_layer_desc *layers, int32_t nlayers,
                    int32_t loss_kind, const gn_adam_desc *adam, int32_t max_batch,
                    int32_t workers, gn_model **out);
void gn_model_destroy(gn_model *m);
int gn_model_nparams(gn_model *m, int64_t *n);
int gn_model_layer_params(gn_model *m, int32_t layer, int64_t *offset, int64_t *count);
int gn_model_out_size(gn_model *m, int32_t *n);
/* The layers as built (a loaded model's descriptions) and the loss. */
int gn_model_layer_count(gn_model *m, int32_t *n);
int gn_model_layer_desc(gn_model *m, int32_t layer, gn_layer_desc *out);
int gn_model_loss_kind(gn_model *m, int32_t *loss_kind);
/* Network.Params / SetParams / Gradients (net.go:549-572, 787-846). */
int gn_model_get_params(gn_model *m, float *dst, int64_t offset, int64_t n);
int gn_model_set_params(gn_model *m, const float *src, int64_t offset, int64_t n);
int gn_model_get_grads(gn_model *m, float *dst, int64_t offset, int64_t n);
int gn_model_get_adam(gn_model *m, float *m_dst, float *v_dst, int64_t offset, int64_t n,
                      int32_t *timestep);
/* Restores Adam moments and the timestep (resume; the reference's
 * Adam.NewStep / StepInPlace state, opt.go:237-335). */
int gn_model_set_adam(gn_model *m, const float *m_src, const float *v_src, int64_t offset, int64_t n,
                      int32_t timestep);
/* Device pointers of the arena regions (for zero-copy callers). */
int gn_model_arena(gn_model *m, float **params, float **grads, float **adam_m, float **adam_v);

/* Network.TrainBatch (net.go:412-436): one fwd+bwd over B samples, gradient
 * average, Adam step.  Host inputs: x is B x in_size, y is B x out_size
 * (row major, the [][]float32 batches flattened).  loss_out may be NULL.
 * On failure: a step that failed before any parameter was updated leaves
 * the model as it was.  Large models update each layer as soon as its
 * backward is done; a step of such a model that fails after some layers
 * were updated leaves those at step t and the others at t-1 (reload a
 * checkpoint), with the Adam timestep at t, so a retry never applies bias
 * correction t twice. */
int gn_model_train_step(gn_model *m, const float *x, const float *y, int32_t B, float *loss_out);
/* Same with HBM-resident x / y; the mean loss stays on the device (read it
 * with gn_model_read_loss).  No host synchronisation. */
int gn_model_train_step_device(gn_model *m, const float *x_dev, const float *y_dev, int32_t B);
/* No counterpart in the reference (launch-overhead control).  Training steps
 * of models without MoE or LSTM layers replay their forward + loss + backward
 * launches from a HIP graph: the first step for a given (x, y, B, training
 * flags) runs eagerly, the second is captured, later ones replay it; Adam is
 * launched after it as usual.  Same kernels, same results.  on = 0 turns it
 * off (and frees the graphs), 1 back on (the default).  A model keeps at most
 * 4 graphs; gn_model_reserve frees them.  A replay reads x and y at the
 * addresses of the step it was captured from, which are the addresses its
 * key matched. */
int gn_model_set_graphs(gn_model *m, int32_t on);
/* Number of captured step graphs the model holds. */
int gn_model_graph_count(gn_model *m, int32_t *n);
/* Test hook (no counterpart in the reference): polls per wait of the
 * cooperative LSTM BPTT kernel before it reports a timeout (default 2^18);
 * a negative value makes every wait time out at once, so the error path
 * (GN_ERR_HIP at the next gn_model_read_loss / gn_model_train_step) can be
 * tested without a fault. */
int gn_debug_lstm_spin_limit(gn_model *model, int32_t polls);
/* Test hook (no counterpart in the reference): polls of the LSTM clip
 * kernel's wait for the Gram kernel it runs beside (default 2048).  When the
 * two kernels do not run at the same time (a profiler, a busy device) the
 * clip gives up after that many polls and a launch queued after the Gram
 * kernel clips the chain instead; 0 forces that path, whose results equal
 * the overlapped path's bit for bit. */
int gn_debug_lstm_clip_bail(gn_model *model, int32_t polls);
/* Test hook (no counterpart in the reference): on = 0 makes training passes
 * run the output Dense layer through its GEMMs, loss-row and column-sum
 * kernels even where it qualifies for the two fused output-layer kernels
 * (at most 32 outputs, input width a multiple of 4); 1 (the default) allows
 * them.  Both paths compute the same step to float32 rounding. */
int gn_debug_fused_tail(gn_model *model, int32_t on);
/* Test hook (no counterpart in the reference): on = 0 makes train steps of
 * small models (under 8 Mi parameters) run Network.Step's Adam update as a
 * launch of its own after the backward; 1 (the default) lets the backward's
 * last launch carry it where that launch writes the step's last gradients
 * (a first Conv2D's weight-gradient reduction).  Both give the same step bit
 * for bit. */
int gn_debug_step_update(gn_model *model, int32_t on);
/* Test hook (no counterpart in the reference): on = 1 runs the backward's
 * parameter-gradient kernels (Dense dW and bias sums, the transformer
 * block's token sums and weight gradients) on a second stream beside the
 * input-gradient kernels, as steps with per-layer Adam updates (models of
 * at least 8 Mi parameters) always do; 0 (the default) keeps them on the
 * main stream otherwise.  Both give the same step bit for bit. */
int gn_debug_side_streams(gn_model *model, int32_t on);
/* Forward + backward + average only (grads valid, no Adam step). */
int gn_model_accumulate_device(gn_model *m, const float *x_dev, const float *y_dev, int32_t B);
/* Network.Step (net.go:260-284): Adam.NewStep + StepInPlace on the arena. */
int gn_model_step(gn_model *m);
int gn_model_read_loss(gn_model *m, float *loss);
/* Sequential.Predict / PredictBatch (sequential.go:118-160): inference mode
 * forward of B samples; out is B x out_size. */
int gn_model_predict(gn_model *m, const float *x, int32_t B, float *out);
/* The same with HBM-resident x (B x in_size) and output (B x out_size); no
 * host synchronisation (the device-side ForwardBatch of sequential.go:145-160). */
int gn_model_predict_device(gn_model *m, const float *x_dev, int32_t B, float *out_dev);
/* Network.SetTraining (net.go:187-193): sets the flag of every layer.  Layers
 * start as the reference constructs them (Dropout and BatchNorm2D in training
 * mode, MoE not: dropout.go:56, batchnorm2d.go:88, moe.go:46-90); Predict
 * turns the flags off and leaves them off (sequential.go:118-134).  With
 * workers > 1 a training step uses the flags of trainBatchParallel's worker
 * clones, which copy the network's flags when first needed and keep them
 * (net.go:129-152). */
int gn_model_set_training(gn_model *m, int32_t training);
int gn_model_get_training(gn_model *m, int32_t layer, int32_t *training);
/* Network.TrainBatch / PredictBatch accept any batch size (net.go:412-436):
 * grows the batch-sized buffers to max_batch samples, keeping parameters,
 * gradients, Adam state, running statistics, noise streams and flags.  A
 * smaller value is a no-op.  On failure the model keeps its old size. */
int gn_model_reserve(gn_model *m, int32_t max_batch);
/* Samples the last training step skipped because an Embedding index was out
 * of range: the reference's batch loop drops such a sample (net.go:738-741;
 * a trainBatchParallel worker drops the rest of its chunk and the chunk's
 * loss, net.go:641-655) and the step still applies.  Inference passes report
 * the same condition as GN_ERR_INDEX (ForwardBatch returns the error,
 * net.go:447-450). */
int gn_model_skipped_samples(gn_model *m, int32_t *count);
/* Layer probes for parity tests: saved output of `layer` for the last batch
 * (B x out_len); int32 indices of the last batch: MaxPool2D argmax switches
 * (B x out_len) or the MoE routes (B x k expert ids, routing order). */
int gn_model_layer_output(gn_model *m, int32_t layer, float *dst, int64_t n);
int gn_model_layer_argmax(gn_model *m, int32_t layer, int32_t *dst, int64_t n);
/* BatchNorm2D running statistics (C floats each) of `layer`:
 * GetRunningMean / GetRunningVar (batchnorm2d.go:837-838) and, for restoring
 * a checkpoint, writing them back (NamedParams running_mean / running_var,
 * batchnorm2d.go:755-767). */
int gn_model_get_running_stats(gn_model *m, int32_t layer, float *mean, float *var, int32_t n);
int gn_model_set_running_stats(gn_model *m, int32_t layer, const float *mean, const float *var,
                               int32_t n);

/* ---- checkpoints: the formats either side of training ------------------
 * Network.SaveBinaryWeights (net.go:1119-1214): "GONN", int32 version 1,
 * int32 tensor count, then per tensor int32 name length, name, int32 rank,
 * int32 shape[rank], int32 length, float32 data (little endian).  Tensors
 * are each layer's NamedParams (or its flat Params) named
 * layer_<i>_<ExtractLayerConfig type>_<name> (net.go:1425-1505). */
int gn_model_save_binary_weights(gn_model *m, const char *path);
/* Reads a SaveBinaryWeights file into this model's parameters and
 * BatchNorm2D running statistics; every tensor's name and length must match.
 * (The reference writes the format but has no reader.) */
int gn_model_load_binary_weights(gn_model *m, const char *path);
/* Network.SaveGGUF / SaveGGUFExt (net.go:1217-1392, gguf.go): GGUF v3 with
 * F32 tensors (f16 = 0) or F16 (f16 = 1, Float32ToFloat16's truncation). */
int gn_model_save_gguf(gn_model *m, const char *path, int32_t f16);
/* The whole training state for resume: parameters, Adam moments and
 * timestep, BatchNorm2D running statistics, MoE noise stream states.  No
 * counterpart in the reference, whose gob Save (net.go:863-1006) keeps no
 * Adam moments. */
int gn_model_save_state(gn_model *m, const char *path);
int gn_model_load_state(gn_model *m, const char *path);
/* Network.Save (net.go:863-871, Encode :1008-1075): "GONN", int32 1, then a
 * gob stream of int32(layers), the loss name, "Adam", one LayerConfig per
 * layer (ExtractLayerConfig, net.go:1393-1505), the flat parameters and
 * Adam's GobState (opt.go:262-322: its moments only when the network has at
 * most 1000 parameters, opt.go:129-153).  Byte for byte what a Go process
 * writes when Save is its first use of gob (gob numbers types per process). */
int gn_model_save_gob(gn_model *m, const char *path);
/* net.Load (net.go:875-1005): the reference's checks (magic, version, at
 * most 1000 layers, at most 256M parameters, the parameter count), then its
 * layers rebuilt with their saved parameters, value activations, the saved
 * loss and a fresh Adam(0.001) (the reference never restores the saved
 * optimizer state).  in_len is the input length per sample, needed when the
 * first layer is not Dense or Dropout (0 = from the file).  loss_kind
 * receives GN_LOSS_*.  Layer types, losses and optimizers this library does
 * not build are GN_ERR_UNSUPPORTED, as is a saved parameter count that
 * differs from the layer its config describes. */
int gn_model_load_gob(gn_ctx *ctx, const char *path, int32_t in_len, int32_t max_batch, int32_t workers,
                      gn_model **out, int32_t *loss_kind);

/* ---- per-layer operators on device pointers -----------------------------
 * Batched stand-ins for the per-sample Layer.Forward / Backward calls and the
 * Metal entry points listed next to each. */

/* matMulFusedPersistent + bias_activation (metal_ops.m:1235-1249, 171-195) /
 * Dense.ForwardWithArena (layer.go:346-456): out[b,o] = act(b[o] + x[b,:].W[o,:]).
 * Softmax/LogSoftmax pointers apply the row activation. */
int gn_dense_forward(gn_ctx *ctx, const float *x, const float *W, const float *bias, float *out,
                     int32_t B, int32_t in, int32_t out_n, int32_t act, int32_t act_is_ptr);
/* Dense.Backward (layer.go:488-667) for a batch: dz from gout and the saved
 * output, gradW = scale*dz^T x, gradB = scale*colsum(dz) (overwrite), and
 * gin = dz W when gin != NULL. */
int gn_dense_backward(gn_ctx *ctx, const float *x, const float *W, const float *out,
                      const float *gout, float *gradW, float *gradB, float *gin, float *dz_scratch,
                      int32_t B, int32_t in, int32_t out_n, int32_t act, int32_t act_is_ptr,
                      float scale);
/* No counterpart in the reference: gn_dense_backward for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments without the dz workspace;
 * dz and the partial sums live in a static 32 MiB device array of the
 * library (one per GPU, held until the process ends), so B x out_n may not
 * exceed 4,194,304 floats (GN_ERR_INVALID otherwise).  The call allocates
 * nothing.  Calls that overlap on one GPU share that array and race: the
 * caller serialises them. */
int gn_dense_backward_noalloc(gn_ctx *ctx, const float *x, const float *W, const float *out,
                              const float *gout, float *gradW, float *gradB, float *gin, int32_t B,
                              int32_t in, int32_t out_n, int32_t act, int32_t act_is_ptr, float scale);

/* Common to the operators below: B samples, each in the layer's flat
 * per-sample layout (its InSize / OutSize), row-major; parameter gradients
 * are written, not accumulated, and multiplied by `scale` (1/B gives the
 * batch average of Network.TrainBatch); an input gradient is written when its
 * pointer is not NULL.  Calls queue work on the context's stream. */

/* Conv2D.ForwardWithArena (conv2d.go:716-960, Metal conv path metal.go:6-50):
 * out = act(conv(x, W) + b) per sample, NCHW, params = [W (outC x inC x k x k)
 * | b (outC)] as Conv2D.Params().  act: scalar GN_ACT_* (Softmax not allowed). */
int gn_conv2d_forward(gn_ctx *ctx, const float *x, const float *params, float *out, int32_t B,
                      int32_t inC, int32_t H, int32_t W, int32_t outC, int32_t k, int32_t stride,
                      int32_t pad, int32_t act);
/* Conv2D.Backward (conv2d.go:997-1236) over the batch: dz = gout * act'(out),
 * grads = [dW | db] = scale * batch sums, gin = col2im(W^T dz). */
int gn_conv2d_backward(gn_ctx *ctx, const float *x, const float *params, const float *out,
                       const float *gout, float *grads, float *gin, int32_t B, int32_t inC,
                       int32_t H, int32_t W, int32_t outC, int32_t k, int32_t stride, int32_t pad,
                       int32_t act, float scale);
/* MaxPool2D.ForwardWithArena (maxpool2d.go:106-226; MaxPool2DPersistent
 * metal.go:343): first strict maximum of each window, padding never wins;
 * argmax = the winner's flat index inside its sample (int32, one per output). */
int gn_maxpool2d_forward(gn_ctx *ctx, const float *x, float *out, int32_t *argmax, int32_t B,
                         int32_t C, int32_t H, int32_t W, int32_t k, int32_t stride, int32_t pad);
/* MaxPool2D.Backward (maxpool2d.go:357-411): gin[i] = sum of gout over the
 * outputs whose argmax is i (every gin element is written). */
int gn_maxpool2d_backward(gn_ctx *ctx, const float *gout, const int32_t *argmax, float *gin,
                          int32_t B, int32_t C, int32_t H, int32_t W, int32_t k, int32_t stride,
                          int32_t pad);
/* Dropout.ForwardWithArena (dropout.go:85-155): in training mode mask (n
 * floats) receives the first n draws of RNG(42) against p (Reset reseeds the
 * stream before every sample, dropout.go:399-401, so every sample shares it)
 * and out = x * mask / (1 - p); in inference mode out = x. */
int gn_dropout_forward(gn_ctx *ctx, const float *x, float *out, float *mask, int32_t B, int32_t n,
                       float p, int32_t training);
/* Dropout.Backward (dropout.go:241-293): gin = gout * mask / (1 - p) in
 * training mode, gout otherwise. */
int gn_dropout_backward(gn_ctx *ctx, const float *gout, const float *mask, float *gin, int32_t B,
                        int32_t n, float p, int32_t training);
/* Output layer and loss: zo (B x C pre-activations) receives act(zo) (Softmax
 * / LogSoftmax rows when act_is_ptr, layer.go:183-205), loss_rows the
 * per-sample loss (MSE / CrossEntropy Forward, loss.go:53-70, 120-145) and dz
 * the gradient at the pre-activations (loss BackwardInPlace loss.go:91-112,
 * 165-185, then Dense's activation backward layer.go:488-567, Softmax
 * Jacobian included). */
int gn_softmax_ce_backward(gn_ctx *ctx, float *zo, const float *y, float *dz, float *loss_rows,
                           int32_t B, int32_t C, int32_t act, int32_t act_is_ptr, int32_t loss_kind);
/* LayerNorm.ForwardWithArena (layernorm.go:193-306) over `rows` rows of N:
 * y = gamma (x - mean) / std + beta, std = sqrt(var + eps) (eps 0 selects
 * 1e-5); stats = (mean, std) per row, kept for the backward. */
int gn_layernorm_forward(gn_ctx *ctx, const float *x, const float *gamma, const float *beta,
                         float *y, float *stats, int32_t rows, int32_t N, float eps);
/* LayerNorm.Backward (layernorm.go:334-441): dx by the reference's formula
 * (its last term divides by N std^2), dgamma = scale * sum g * xhat, dbeta =
 * scale * sum g; work = rows x N floats of scratch. */
int gn_layernorm_backward(gn_ctx *ctx, const float *g, const float *x, const float *gamma,
                          const float *stats, float *dx, float *dgamma, float *dbeta, float *work,
                          int32_t rows, int32_t N, float scale);
/* MultiHeadAttention (transformer.go:277-776): x is B x T x D, params = [wQ |
 * wK | wV | wOut], each a Linear Dense (W D x D, b D).  work carries the
 * forward's saved state to the backward: gn_mha_workspace floats, the same
 * buffer and x for both calls.  Any T and head size: up to T = 128 and
 * 32-wide heads in fused kernels, beyond that through batched GEMMs over the
 * materialised B x heads x T x T scores (included in the workspace); B x heads
 * must not exceed 65535. */
int gn_mha_workspace(int32_t B, int32_t T, int32_t D, int32_t heads, int32_t use_rope,
                     int64_t *floats);
/* MultiHeadAttention.ForwardWithArena (transformer.go:405-529): Q, K, V per
 * token, RoPE on Q and K when use_rope (applyRoPE transformer.go:212-236),
 * softmax(Q K^T / sqrt(hd)) V per head (causal mask -1e9), out = wOut(O). */
int gn_mha_forward(gn_ctx *ctx, const float *x, const float *params, float *out, float *work,
                   int32_t B, int32_t T, int32_t D, int32_t heads, int32_t causal, int32_t use_rope);
/* MultiHeadAttention.Backward (transformer.go:557-690): each projection's
 * weight gradient uses its last token's input (the per-token Dense layers
 * keep only the last Forward's input) and its bias gradient sums every
 * token; conjugate rotation before wQ / wK; gin = sum of the three
 * projections' input gradients. */
int gn_mha_backward(gn_ctx *ctx, const float *x, const float *params, const float *gout,
                    float *grads, float *gin, float *work, int32_t B, int32_t T, int32_t D,
                    int32_t heads, int32_t causal, int32_t use_rope, float scale);
/* SequenceUnroller(LSTM) with return_sequences false (unroller.go:57-213,
 * lstm.go:144-753): x is B x T x I, params = [Wx (4H x I) | Wh (4H x H) | b
 * (4H)], gates i, f, g, o; out = h_{T-1} (B x H); hidden <= 1024.  work:
 * gn_lstm_workspace floats (the same B, T, I, H, workers for both calls). */
int gn_lstm_workspace(int32_t B, int32_t T, int32_t I, int32_t H, int32_t workers,
                      int64_t *floats);
/* LSTM.ForwardWithArena per step (lstm.go:276-442): only the input gate adds Wx x +
 * Wh h to its bias (lstmComputeInputGates, lstm.go:1065-1101). */
int gn_lstm_seq_forward(gn_ctx *ctx, const float *x, const float *params, float *out, float *work,
                        int32_t B, int32_t T, int32_t I, int32_t H, int32_t return_sequences);
/* SequenceUnroller.Backward + LSTM.Backward per step (unroller.go:133-213,
 * lstm.go:476-699, clipGradients 725-753): carried dh (dh_{t-1} = dh_t + Wh^T dG), dWx from the last
 * step's input, each worker chain's cumulative gradient clipped to norm 1
 * after every step (`workers` chains of ceil(B / workers) samples, as
 * trainBatchParallel's chunks), gin_t = Wx^T dG_t (unclipped).  return_sequences
 * (NewSequenceUnroller's flag, unroller.go:21-43): out / gout hold every step's
 * h (B x T x H) instead of the last (B x H). */
int gn_lstm_seq_backward(gn_ctx *ctx, const float *x, const float *params, const float *gout,
                         float *grads, float *gin, float *work, int32_t B, int32_t T, int32_t I,
                         int32_t H, int32_t workers, float scale, int32_t return_sequences);
/* Embedding.ForwardWithArena (embedding.go:79-141): x = B x T ids as floats,
 * out = rows of E (V x D), ids = the int32 indices for the backward; bad
 * (optional, B ints) = 1 for a sample with an id outside [0, V), which the
 * reference's Forward rejects (its output rows read row 0 here). */
int gn_embedding_forward(gn_ctx *ctx, const float *x, const float *E, float *out, int32_t *ids,
                         int32_t *bad, int32_t B, int32_t T, int32_t V, int32_t D);
/* Embedding.Backward (embedding.go:147-183) over a batch: Backward zeroes the
 * table's gradient before adding a sample's rows, so gradE = scale * the rows
 * of the last sample of each worker chunk (`workers` chunks of ceil(B /
 * workers); with bad, the last sample the reference's loop still reaches).
 * Contributing rows (chunks x T) above 2048 take a list in the context's
 * scratch (2 ints per row; GN_ERR_UNSUPPORTED beyond 8M rows). */
int gn_embedding_backward(gn_ctx *ctx, const float *gout, const int32_t *ids, const int32_t *bad,
                          float *gradE, int32_t B, int32_t T, int32_t V, int32_t D, int32_t workers,
                          float scale);

/* AvgPool2D.ForwardWithArena / Backward (avgpool2d.go:137-474): B samples of
 * C x H x W, k x k windows, stride, zero padding not counted in the mean. */
int gn_avgpool2d_forward(gn_ctx *ctx, const float *x, float *out, int32_t B, int32_t C, int32_t H,
                         int32_t W, int32_t k, int32_t stride, int32_t pad);
int gn_avgpool2d_backward(gn_ctx *ctx, const float *gout, float *gin, int32_t B, int32_t C, int32_t H,
                          int32_t W, int32_t k, int32_t stride, int32_t pad);
/* RMSNorm.ForwardWithArena / Backward (rmsnorm.go:222-329) over `rows` rows of
 * N: y = gamma x / rms, rms per row for the backward (eps 0 selects 1e-5);
 * dx (may be NULL) follows the reference's formula; dgamma = scale * sums;
 * work: rows x N floats. */
int gn_rmsnorm_forward(gn_ctx *ctx, const float *x, const float *gamma, float *y, float *rms,
                       int32_t rows, int32_t N, float eps);
int gn_rmsnorm_backward(gn_ctx *ctx, const float *g, const float *x, const float *gamma, const float *rms,
                        float *dx, float *dgamma, float *work, int32_t rows, int32_t N, float scale);
/* SwiGLU.ForwardWithArena / Backward (swiglu.go:103-232): params = [W | V]
 * (out x in each, no biases), y = swish(W x) * (V x); grads = [dW | dV]
 * written (scale * sums); gin may be NULL; work: gn_swiglu_workspace floats
 * shared by the forward and backward of one batch. */
int gn_swiglu_workspace(int32_t B, int32_t out, int64_t *floats);
int gn_swiglu_forward(gn_ctx *ctx, const float *x, const float *params, float *out, float *work, int32_t B,
                      int32_t in, int32_t out_size);
int gn_swiglu_backward(gn_ctx *ctx, const float *x, const float *params, const float *gout, float *grads,
                       float *gin, float *work, int32_t B, int32_t in, int32_t out_size, float scale);
/* BatchNorm2D.ForwardWithArena / Backward (batchnorm2d.go:255-666): B samples
 * of C x HW; params = [gamma | beta] or NULL (affine = false).  training:
 * each sample normalised by its own channel statistics (the reference runs one
 * sample per Forward), running mean / var advanced once per sample in sample
 * order; stats = 3 B C floats (mean, var, std) for the backward.  Inference
 * uses the running statistics; its backward gives dx only and zero parameter
 * gradients (batchnorm2d.go:525-551).  work: 2 B C floats. */
int gn_batchnorm2d_forward(gn_ctx *ctx, const float *x, const float *params, float *out, float *stats,
                           float *running_mean, float *running_var, int32_t B, int32_t C, int32_t HW,
                           float eps, float momentum, int32_t training);
int gn_batchnorm2d_backward(gn_ctx *ctx, const float *gout, const float *x, const float *params,
                            const float *stats, const float *running_var, float *grads, float *gin,
                            float *work, int32_t B, int32_t C, int32_t HW, float eps, int32_t training,
                            float scale);
/* SequenceUnroller(GRU) forward / backward (unroller.go:57-213,
 * gru.go:192-703): x = B x T x I, params = [Wx (3H x I) | Wh (2H x H) | b
 * (3H)], the reference's quirks kept (candidate weighted by 1 - u in the
 * backward, no reset-gate delta, dWx from the last step's input, carried dh);
 * return_sequences: out / gout hold every step's h.  work: gn_gru_workspace
 * floats, shared by the forward and backward of one batch. */
int gn_gru_workspace(int32_t B, int32_t T, int32_t I, int32_t H, int64_t *floats);
int gn_gru_seq_forward(gn_ctx *ctx, const float *x, const float *params, float *out, float *work, int32_t B,
                       int32_t T, int32_t I, int32_t H, int32_t return_sequences);
int gn_gru_seq_backward(gn_ctx *ctx, const float *x, const float *params, const float *gout, float *grads,
                        float *gin, float *work, int32_t B, int32_t T, int32_t I, int32_t H, float scale,
                        int32_t return_sequences);
/* MoE.ForwardWithArena / Backward (moe.go:140-313): params = [gating W (E x
 * I), b | per expert W (O x I), b]; the top K experts by gate softmax
 * (stable in index order for ties), LeakyReLU(0.1) experts.  training adds
 * the layer's RNG gate noise: *noise is the stream's state (42 at
 * construction), advanced by E draws per sample; and the load-balancing
 * gradient.  work: gn_moe_workspace floats, shared by the forward and
 * backward of one batch. */
int gn_moe_workspace(int32_t B, int32_t I, int32_t O, int32_t E, int32_t K, int64_t *floats);
int gn_moe_forward(gn_ctx *ctx, const float *x, const float *params, float *out, float *work, int32_t B,
                   int32_t I, int32_t O, int32_t E, int32_t K, int32_t training, uint64_t *noise);
int gn_moe_backward(gn_ctx *ctx, const float *x, const float *params, const float *gout, float *grads,
                    float *gin, float *work, int32_t B, int32_t I, int32_t O, int32_t E, int32_t K,
                    int32_t training, float scale);

/* Generic fp32 MFMA GEMM: C[M,N] = alpha * op(A) op(B); trans flags as BLAS
 * (A is M x K row-major when transA == 0, K x M when 1; B is K x N when
 * transB == 0, N x K when 1).  Stands in for matMulMPSPersistent
 * (metal_ops.m:1220-1233). */
int gn_gemm(gn_ctx *ctx, int32_t transA, int32_t transB, int32_t M, int32_t N, int32_t K,
            float alpha, const float *A, int32_t lda, const float *B, int32_t ldb, float *C,
            int32_t ldc);
/* Adam.StepInPlace (opt.go:207-252) over n elements of the flat arena, with
 * the optimizer timestep already advanced (first Network.Step => 1). */
int gn_adam_step(gn_ctx *ctx, float *params, const float *grads, float *m, float *v, int64_t n,
                 float lr, float beta1, float beta2, float eps, int32_t timestep);

/* ---- kernel timing (measurement hook; no reference counterpart) ---------
 * While enabled, every kernel launch of the library is bracketed by HIP events
 * on the context stream and attributed to a class.  gn_timing_report
 * synchronises the stream and returns the launch count and summed kernel time
 * of a class since the last enable. */
#define GN_KCLASS_GEMM 0   /* gemm_f32_mfma (Dense fwd / dX / dW) */
#define GN_KCLASS_ADAM 1   /* adam_kernel */
#define GN_KCLASS_OTHER 2  /* row kernels, column sums, dropout, ... */
int gn_timing_enable(gn_ctx *ctx, int enable);
int gn_timing_report(gn_ctx *ctx, int kclass, int64_t *launches, double *total_ms);
/* Per kernel (or fused launch group) since the last enable: name, class,
 * launch count, summed time and summed algorithmic work -- bytes moved for a
 * memory-bound kernel (compulsory fp32 reads and writes), FLOPs for a GEMM /
 * matrix-core kernel -- so units / time is its achieved GB/s or FLOP/s.
 * Writes at most cap entries and the number of distinct names to *n. */
typedef struct gn_kernel_stat {
  char name[48];
  int32_t cls;      /* GN_KCLASS_* */
  int64_t launches;
  double ms;
  double units;
} gn_kernel_stat;
int gn_timing_kernels(gn_ctx *ctx, gn_kernel_stat *out, int32_t cap, int32_t *n);
/* The launch floor the per-kernel times are read against: reps launches of an
 * empty kernel of `blocks` 256-thread workgroups on the context stream, timed
 * like every library launch (recorded as "floor" while timing is enabled). */
int gn_timing_floor(gn_ctx *ctx, int32_t blocks, int32_t reps);

/* ---- synthetic inputs (host side; harness utility) ----------------------
 * The reference's LCG (layer.go:61-81): U[0,1) stream, N(0,1) by one
 * Box-Muller cosine per two draws (u1 clamped to 1e-7, f64 math), class ids
 * floor(U*nclass) clamped to nclass-1. */
int gn_fill_uniform(float *dst, int64_t n, uint64_t seed);
int gn_fill_normal(float *dst, int64_t n, uint64_t seed);
int gn_fill_class_ids(int32_t *dst, int64_t n, int32_t nclass, uint64_t seed);

#ifdef __cplusplus
}
#endif
#endif /* GONEURON_HIP_H */
