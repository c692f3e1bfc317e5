/*
 * refcpu — CPU restatement of GoNeuron's pure-Go float32 training step.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity oracle: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only
 * as the checker or the timed CPU baseline.  The product (libgoneuron_hip.so)
 * never links, loads or calls it.
 *
 * It follows the reference per-sample algorithm line by line (file:line
 * citations point into the GoNeuron tree):
 *   Network.trainBatchSequential      internal/net/net.go:721-784
 *   Network.trainBatchParallel        internal/net/net.go:588-717 (W workers)
 *   Dense                             internal/layer/layer.go:224-667
 *   matMulOptimized (summation order) internal/layer/matmul_optimized.go:18-152
 *   activations                       internal/activations/activations.go:22-236,345-352
 *   CrossEntropy / MSE                internal/loss/loss.go:53-178
 *   Adam                              internal/opt/opt.go:117-258
 *   Dropout                           internal/layer/dropout.go:47-401
 *   Conv2D                            internal/layer/conv2d.go:114-1174
 *   MaxPool2D                         internal/layer/maxpool2d.go:106-410,508-513
 *   AvgPool2D                         internal/layer/avgpool2d.go:98-220,401-474,560-565
 *   RMSNorm                           internal/layer/rmsnorm.go:73-96,222-240,301-335
 *   SwiGLU                            internal/layer/swiglu.go:73-232
 *   BatchNorm2D                       internal/layer/batchnorm2d.go:103-135,255-511,524-665
 *   GRU (in a SequenceUnroller)       internal/layer/gru.go:110-510, unroller.go:57-213
 *   MoE                               internal/layer/moe.go:47-313, net.go:129-152 (worker clones)
 *   Flatten                           internal/layer/reshape.go:64-96
 *   LSTM                              internal/layer/lstm.go:144-751,1065-1101
 *   SequenceUnroller                  internal/layer/unroller.go:57-213
 *   Embedding                         internal/layer/embedding.go:42-183
 *   PositionalEncoding                internal/layer/transformer.go:51-120
 *   MultiHeadAttention                internal/layer/transformer.go:318-690
 *   TransformerBlock                  internal/layer/transformer.go:908-1279
 *   LayerNorm                         internal/layer/layernorm.go:83-441
 *   CLSPooling                        internal/layer/transformer.go:1679-1725
 *   RNG                               internal/layer/layer.go:61-81
 * Built with -O2 -ffp-contract=off (Go amd64 GOAMD64=v1 emits no FMA).
 */
#ifndef GN_REFCPU_H
#define GN_REFCPU_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Activation object kinds (activations.go).  `is_ptr` mirrors Go's value vs
 * pointer receiver distinction that cacheActivationType (layer.go:183-205)
 * depends on. */
enum {
  GNO_ACT_NIL = 0,
  GNO_ACT_RELU = 1,
  GNO_ACT_SIGMOID = 2,
  GNO_ACT_TANH = 3,
  GNO_ACT_SOFTMAX = 4,
  GNO_ACT_LOGSOFTMAX = 5,
  GNO_ACT_LINEAR = 6,
  GNO_ACT_GELU = 7,
  GNO_ACT_LEAKYRELU = 8, /* NewLeakyReLU(0.1): a pointer (ActTypeLeakyReLU) */
};

enum {
  GNO_LAYER_DENSE = 1,
  GNO_LAYER_DROPOUT = 2,
  GNO_LAYER_CONV2D = 3,
  GNO_LAYER_MAXPOOL2D = 4,
  GNO_LAYER_FLATTEN = 5,
  GNO_LAYER_EMBEDDING = 6,
  GNO_LAYER_POSENC = 7,
  GNO_LAYER_TRANSFORMER = 8,
  GNO_LAYER_CLSPOOL = 9,
  GNO_LAYER_LSTM_UNROLLER = 10,
  GNO_LAYER_AVGPOOL2D = 11,
  GNO_LAYER_RMSNORM = 12,
  GNO_LAYER_SWIGLU = 13,
  GNO_LAYER_BATCHNORM2D = 14,
  GNO_LAYER_GRU_UNROLLER = 15,
  GNO_LAYER_MOE = 16,
  GNO_LAYER_MHA = 17,       /* MultiHeadAttention alone (dim, num_heads, seq_len, causal, use_rope) */
  GNO_LAYER_LAYERNORM = 18, /* LayerNorm alone (dim = normalizedShape, in_size = sample length, eps) */
  GNO_LAYER_GAP1D = 19,     /* GlobalAveragePooling1D (seq_len, dim) */
};

enum { GNO_LOSS_MSE = 1, GNO_LOSS_CE = 2 };

typedef struct gno_layer_spec {
  int32_t kind;
  int32_t in_size;      /* Dense in / Dropout size / Flatten size / LSTM input */
  int32_t out_size;     /* Dense out / LSTM hidden */
  int32_t act;          /* GNO_ACT_* */
  int32_t act_is_ptr;   /* 1: &activations.X{} ; 0: activations.X{} value */
  int32_t in_channels;  /* Conv2D / MaxPool2D (-1 = lazy) */
  int32_t out_channels;
  int32_t kernel, stride, padding;
  float p;              /* Dropout */
  int32_t seq_len, num_heads, ff_dim, causal, vocab, dim; /* RMSNorm: dim = normalizedShape */
  int32_t return_sequences;
  float eps;            /* RMSNorm eps (0 = 1e-5) */
  int32_t block_act;    /* TransformerBlock ff1: 0 ReLU, 1 SwiGLU, 2 GELU (transformer.go:199-203) */
  int32_t block_norm;   /* TransformerBlock norms: 0 LayerNorm, 1 RMSNorm (transformer.go:205-210) */
  int32_t use_rope;     /* TransformerBlock attention: rotary embeddings on Q and K */
  float momentum;       /* BatchNorm2D running-stat momentum (the facade's 0.1) */
  int32_t no_affine;    /* BatchNorm2D without gamma / beta */
  int32_t num_experts, top_k; /* MoE */
} gno_layer_spec;

typedef struct gno_net gno_net;

/* LCG (layer.go:61-81). */
float gno_rand_float(uint64_t *state);
/* Synthetic data: uniform U[0,1) stream, N(0,1) Box-Muller pairs, class ids. */
void gno_fill_uniform(float *dst, int64_t n, uint64_t seed);
void gno_fill_normal(float *dst, int64_t n, uint64_t seed);
void gno_fill_class_ids(int32_t *dst, int64_t n, int32_t nclass, uint64_t seed);

gno_net *gno_net_create(const gno_layer_spec *specs, int32_t nlayers,
                        int32_t loss_kind, float lr, int32_t workers);
void gno_net_destroy(gno_net *n);
int64_t gno_net_nparams(const gno_net *n);
int64_t gno_net_layer_param_offset(const gno_net *n, int32_t layer);
int64_t gno_net_layer_param_count(const gno_net *n, int32_t layer);
float *gno_net_params(gno_net *n);
float *gno_net_grads(gno_net *n);
float *gno_net_adam_m(gno_net *n);
float *gno_net_adam_v(gno_net *n);
int32_t gno_net_adam_timestep(const gno_net *n);
/* One TrainBatch: x is B x in (row major), y is B x out. Returns mean loss.
 * workers==1 -> trainBatchSequential; >1 -> trainBatchParallel chunking. */
float gno_net_train_batch(gno_net *n, const float *x, const float *y, int32_t B);
/* Same as train_batch but stops before Step (grads hold the averaged batch
 * gradient), for gradient parity checks. */
float gno_net_accumulate_batch(gno_net *n, const float *x, const float *y, int32_t B);
void gno_net_step(gno_net *n);
/* A batch pass with each sample's output gradient given (gout, B x out)
 * instead of a loss (od = output length per sample): outputs into out and
 * input gradients into gin (either
 * may be NULL); parameter gradients accumulated and averaged as by
 * gno_net_accumulate_batch (same worker chunking).  For testing one layer
 * against an arbitrary upstream gradient. */
void gno_net_accumulate_grad(gno_net *n, const float *x, const float *gout, int32_t B, int32_t od,
                             float *out, float *gin);
/* Forward of one sample (training flag as set); writes out, returns out len. */
int32_t gno_net_forward(gno_net *n, const float *x, float *out);
void gno_net_set_training(gno_net *n, int32_t training);
int32_t gno_net_out_size(const gno_net *n);
/* Per-layer probes for unit tests: argmax of a MaxPool2D layer after the last
 * forward (count returned), last saved pre-activation of layer `layer`. */
int32_t gno_net_layer_argmax(gno_net *n, int32_t layer, int32_t *dst, int32_t cap);
/* MoE routes logged since the previous call (the first call starts the log
 * and returns 0): k expert ids per forward in routing order. */
int32_t gno_net_layer_routes(gno_net *n, int32_t layer, int32_t *dst, int32_t cap);
int32_t gno_net_layer_preact(gno_net *n, int32_t layer, float *dst, int32_t cap);

/* Stand-alone kernels of the reference (for golden-vector checks). */
void gno_activate_batch(int32_t act, float *x, int32_t n);            /* softmax/logsoftmax */
float gno_activate(int32_t act, float x);
float gno_derivative(int32_t act, float x);
float gno_loss_forward(int32_t loss_kind, const float *pred, const float *y, int32_t n);
void gno_loss_backward(int32_t loss_kind, const float *pred, const float *y, float *grad, int32_t n);
/* Adam.StepInPlace with the optimizer's timestep already advanced to `timestep`
 * (NewStep increments before the update; opt.go:237-258). */
void gno_adam_step_inplace(float *params, const float *grads, float *m, float *v,
                           int64_t n, float lr, float beta1, float beta2, float eps,
                           int32_t timestep);
/* AvgPool2D forward of one sample (out, returns its length) and, when g and
 * gin are given, the backward of g into gin. */
int32_t gno_avgpool2d(const float *x, int32_t total, int32_t inC, int32_t k, int32_t stride,
                      int32_t pad, float *out, const float *g, float *gin);
/* RMSNorm of one sample (total = rows x n) with the given gamma into out;
 * with g, gin and ggamma also the backward (ggamma accumulates).  Returns the
 * row count, -1 when n does not divide total. */
int32_t gno_rmsnorm(const float *x, int32_t total, int32_t n, float eps, const float *gamma,
                    float *out, const float *g, float *gin, float *ggamma);
/* SwiGLU of one sample with params [W | V] (each out x in) into y; with g,
 * gin and gparams also the backward (gparams accumulates). */
void gno_swiglu(const float *x, int32_t in, int32_t out, const float *params, float *y,
                const float *g, float *gin, float *gparams);
/* applyRoPE over T tokens of nh heads of hd, in place (conj: the inverse). */
void gno_rope(float *x, int32_t T, int32_t nh, int32_t hd, int32_t conj);
/* BatchNorm2D of N samples of C channels x HW positions (x is N*C*HW) with
 * the batch statistics (training, updating rm / rv) or the running ones; with
 * g, gin (and ggamma / gbeta when affine) also the training backward. */
void gno_batchnorm2d(const float *x, int32_t N, int32_t C, int32_t HW, float eps, float momentum,
                     int32_t affine, const float *gamma_beta, int32_t training, float *out,
                     float *rm, float *rv, const float *g, float *gin, float *ggamma_beta);
/* Running mean / var of BatchNorm2D layer li (C each); returns C or 0. */
int32_t gno_net_layer_running_stats(gno_net *n, int32_t li, float *mean, float *var);
/* SequenceUnroller(GRU) of one sample (x: T x I) with params [Wx | Wh | b]:
 * the last hidden state into out (H); with g, gin and gparams the backward
 * (gin: T x I, gparams accumulates). */
void gno_gru_sequence(const float *x, int32_t I, int32_t H, int32_t T, const float *params,
                      float *out, const float *g, float *gin, float *gparams);
/* MoE of one sample with params [gating W, b | expert W, b ...]; *rng is the
 * noise stream state (used and advanced in training mode); active gets the
 * top-k expert ids in routing order; with g, gin and gparams the backward. */
int32_t gno_moe(const float *x, int32_t I, int32_t O, int32_t E, int32_t K, const float *params,
                int32_t training, uint64_t *rng, float *out, int32_t *active, const float *g,
                float *gin, float *gparams);
/* matMulOptimized: out[b,o] = bias[o] + sum_i in[b,i] w[o,i]. */
void gno_matmul(const float *in, const float *w, const float *bias, float *out,
                int32_t batch, int32_t in_size, int32_t out_size);

#ifdef __cplusplus
}
#endif
#endif
