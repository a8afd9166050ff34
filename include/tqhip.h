/* tqhip.h -- C ABI of the MI355X (gfx950) quantized linear-projection library.
 *
 * Drop-in for tiny-llm's kernel dispatch on the quantized-projection path.
 * Reference paths below are relative to the tiny-llm source root.
 *
 * 1. Host-pointer entry points. Exactly the reference's dispatch signatures:
 *    synchronous, caller-owned host buffers, no error return (a HIP failure
 *    prints to stderr and aborts, as the reference's GPU variants do). Weights
 *    are immutable for the life of the process (docs/optimization.md:147-149),
 *    so each weight tensor is copied to HBM once and cached by its host
 *    pointer and byte size; x and y go through a grow-only device workspace.
 *    These are the functions registered as the "hip" variants.
 *
 * 2. Device-pointer entry points (suffix _dev). Same math on buffers already
 *    in HBM, launched asynchronously on `stream` (a hipStream_t; NULL = the
 *    default stream). They return 0 or a negative TQHIP_E* code and never abort.
 *    Scratch: some launches need library-owned device scratch (the split-K
 *    matvec's exchange slots, the prefill GEMM's fp16 copy of X). Each
 *    (device, stream) has its own, grown on demand between launches (the
 *    stream is synchronised first), so calls on different streams never share
 *    it. Under the caller's own stream capture nothing is allocated: a call
 *    that would need more scratch than the stream already has returns
 *    TQHIP_EHIP (run it once eagerly on that stream first), and scratch that a
 *    capture recorded is never freed, so the caller's graph stays valid.
 *
 * 3. Registry. The library carries its own copy of the reference registry for
 *    these families (same names and behaviour, C++ namespace tinyqwen,
 *    tiny-llm_amd/csrc/dispatch.h); the tqhip_set_* / tqhip_dispatch_* symbols
 *    below expose it to C callers.
 *
 * Layouts (runtime/tiny_format.h:58-103, docs/weight_format.md:83-119):
 *   i4 : every row is ceil(in_dim/G) groups of [scale fp16 | zero fp16 | G/2 code bytes],
 *        low nibble = even element; weight = (q - zero) * scale.
 *   VQ2: [codebook 256 x 4 fp16 = 2048 B][out_dim x in_dim/4 uint8 indices], in_dim % 4 == 0.
 *   matmul: X is [K, N] column-major (x[n*K + k]), Y is [M, N] column-major (y[n*M + m]).
 */
#ifndef TQHIP_H
#define TQHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TQHIP_OK 0
#define TQHIP_EBADSHAPE (-1)    /* a dimension < 1, in_dim % 4 != 0 for VQ2, or a null operand pointer
                                   (checked before anything is launched) */
#define TQHIP_EBADGROUP (-2)    /* group_size odd or < 2 */
#define TQHIP_ETOOLARGE (-3)    /* shape exceeds the kernel's 32-bit addressing */
#define TQHIP_ELAUNCH (-4)      /* the kernel launch failed */
#define TQHIP_EFILE (-5)        /* a .tqwen file was unreadable, invalid or of an unsupported kind */
#define TQHIP_EHIP (-6)         /* a HIP allocation or copy failed */
#define TQHIP_ENOSCRATCH (-7)   /* tqhip_matmul_i4_noalloc_dev: the call needs more than the static scratch */

/* ---- 1. host-pointer entry points (the "hip" variants) ------------------ */

/* MatvecI4Fn, kernels/dispatch.h:151-152; replaces matvec_i4_ref (kernels/matvec/matvec_i4_ref.cpp:45). */
void tqhip_matvec_i4(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size);

/* MatvecPairI4Fn, kernels/dispatch.h:162-163 (no i4 pair kernel exists in the reference). */
void tqhip_matvec_pair_i4(const uint8_t *w1, const uint8_t *w2, const float *x, float *y1, float *y2,
                          int out_dim, int in_dim, int group_size);

/* MatvecQkvI4Fn, kernels/dispatch.h:169-171 (no i4 qkv kernel exists in the reference). */
void tqhip_matvec_qkv_i4(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv, const float *x, float *yq,
                         float *yk, float *yv, int q_dim, int kv_dim, int in_dim, int group_size);

/* MatvecVQ2Fn, kernels/dispatch.h:187-188; replaces matvec_vq2_ref (kernels/matvec/matvec_vq2_ref.cpp:52). */
void tqhip_matvec_vq2(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim);

/* MatmulI4Fn, kernels/dispatch.h:249-250; replaces matmul_i4_ref (kernels/matvec/matmul_i4_ref.cpp:53). */
void tqhip_matmul_i4(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size);

/* BiipRotateFn, kernels/dispatch.h:226-227; replaces biip_rotate_activation_ref
 * (kernels/biip/biip_rotate.cpp:37-68): y = blockHadamard((x / scale) * sign),
 * scale == NULL skipping the division, block_size a power of two dividing dim;
 * y may alias x. scale and sign are cached in HBM like weights (by host pointer,
 * size and fingerprint). Bit-identical to the reference's scalar rotation. */
void tqhip_biip_rotate(const float *x, float *y, int dim, const float *scale, const float *sign, int block_size);

/* Drops every cached device copy of host weights (not in the reference: its
 * CUDA variants keep their cache until exit). */
void tqhip_release_weights(void);

/* Timing of the host-pointer calls above (not in the reference; its bench_kernels times the
 * whole call). With timing on, each call records HIP events around its x upload, its
 * kernels and its y download; tqhip_host_timing_last returns the three intervals of the
 * last call in milliseconds (0 until a timed call has run). */
void tqhip_host_timing(int on);
void tqhip_host_timing_last(float *upload_ms, float *kernel_ms, float *download_ms);

/* ---- 2. device-pointer entry points ------------------------------------- */

int tqhip_matvec_i4_dev(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size,
                        void *stream);
int tqhip_matvec_vq2_dev(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, void *stream);
/* The pair and qkv forms (kernels/dispatch.h:162-163, 169-171) on device
 * buffers: one launch covers all the matrices when the staged kernel applies. */
int tqhip_matvec_pair_i4_dev(const uint8_t *w1, const uint8_t *w2, const float *x, float *y1, float *y2, int out_dim,
                             int in_dim, int group_size, void *stream);
int tqhip_matvec_qkv_i4_dev(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv, const float *x, float *yq,
                            float *yk, float *yv, int q_dim, int kv_dim, int in_dim, int group_size, void *stream);
int tqhip_matmul_i4_dev(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size,
                        void *stream);
/* One matrix of a matvec set: its weights, activations, output and shape. */
typedef struct tqhip_i4_mat {
    const uint8_t *w;
    const float *x;
    float *y;
    int out_dim, in_dim;
} tqhip_i4_mat;
/* n independent i4 matvecs y_i = W_i x_i of one group size, each with its own activation
 * vector and shape, for instance a decoder layer's q/k/v/o/gate/up/down (four activation
 * vectors). No counterpart in the reference, whose runtime issues a layer as separate
 * registry calls (runtime/qwen_forward_token.cpp:401, 458, 639, 658 through
 * kernels/dispatch.h:151-175): this is the "matvec set per layer" as one launch. Every
 * matrix with group_size 64, in_dim % 4 == 0, in_dim <= 10240 and x 16-byte aligned goes
 * into one launch per 8 such matrices; any other runs through tqhip_matvec_i4_dev's
 * kernels. Each output has the same bits as the lane kernels of tqhip_matvec_i4_dev give
 * it where those run (rows up to 1024 wide on small grids, up to 6144 wide on very small
 * ones). mats is read during the call. */
int tqhip_matvec_i4_set_dev(const tqhip_i4_mat *mats, int n, int group_size, void *stream);
/* n independent VQ2 matvecs y_i = W_i x_i, each with its own activation vector and shape
 * (tqhip_i4_mat's fields: the weights are a VQ2 tensor, codebook then indices). No
 * counterpart in the reference, whose runtime issues a VQ2 layer as single matvec_vq2 calls
 * (its pair and qkv forms are decompositions, kernels/dispatch.cpp:511-532): this is the
 * "matvec set" for VQ2 as one launch. Every matrix with in_dim % 16 == 0, 4-byte aligned
 * weights and at most 4M lookups (out_dim * in_dim / 4) goes into one launch per 8 such
 * matrices, while a launch holds at most 8M lookups; any other runs alone through
 * tqhip_matvec_vq2_dev's kernels. Each output has the same bits tqhip_matvec_vq2_dev gives
 * it. mats is read during the call. */
int tqhip_matvec_vq2_set_dev(const tqhip_i4_mat *mats, int n, void *stream);
/* tqhip_matmul_i4_dev without any allocation. No counterpart in the reference: this is
 * for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Same kernels and results as
 * tqhip_matmul_i4_dev, bit for bit. X's fp16 copy and the per-token scales (or, at up to
 * 32 tokens with group_size 64, the few-token kernel's partial products) go to a static
 * device array of TQHIP_NOALLOC_SCRATCH_BYTES (16 MiB) that every GPU the library runs on
 * holds until the process ends; its last 64 KiB hold the few-token kernel's tile counters
 * (zero between calls). A call whose fp16 copy needs more than the rest
 * (((ceil(K/64)*64*2*N + 255) & ~255) + 4*N bytes, e.g. above 3261 tokens at K = 2560), or
 * whose few-token partial products do not fit (16 KiB per 128-row tile and K slice, e.g.
 * 151936x896 at up to 32 tokens: 38.9 MB), returns TQHIP_ENOSCRATCH before launching
 * anything; no call is rerouted to another kernel. Group sizes that are not a
 * multiple of 32 run one matvec per token, with kernels that need no scratch. All calls
 * on one GPU share the array: calls that overlap on one GPU (two streams, or two host
 * threads) race and must be ordered by the caller. */
#define TQHIP_NOALLOC_SCRATCH_BYTES (16u << 20)
int tqhip_matmul_i4_noalloc_dev(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size,
                                void *stream);
/* Compact-i4 embedding lookup: out[t][0..dim) = dequant_i4_row(embed, rows[t],
 * dim, group_size, .) for t < n (kernels/ref_ops.h:183-205, called per prompt
 * token by runtime/qwen_forward_prefill.cpp:180); rows is a device array of
 * token ids. Bit-identical to the reference's row decode. */
int tqhip_dequant_i4_rows_dev(const uint8_t *embed, const int *rows, int n, int dim, int group_size, float *out,
                              void *stream);
/* The BiIP rotation on device buffers (y may alias x). */
int tqhip_biip_rotate_dev(const float *x, float *y, int dim, const float *scale, const float *sign, int block_size,
                          void *stream);
/* The portable fp32 one-wave-per-row i4 kernel, used by the fast path for
 * group sizes it does not cover; exported for cross-checks. */
int tqhip_matvec_i4_generic_dev(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim,
                                int group_size, void *stream);

/* ---- 3. registry (kernels/dispatch.h:155-159, 191-195; set_matmul_i4_impl_by_name is new) */

int tqhip_set_matvec_i4_impl_by_name(const char *name);   /* 1 = selected, 0 = unknown name */
const char *tqhip_matvec_i4_impl_name(void);
const char *tqhip_available_matvec_i4_impls(void);
int tqhip_set_matvec_vq2_impl_by_name(const char *name);
const char *tqhip_matvec_vq2_impl_name(void);
const char *tqhip_available_matvec_vq2_impls(void);
int tqhip_set_matmul_i4_impl_by_name(const char *name);
/* The ops registry's BiIP member (set_ops_impl_by_name / ops_impl_name /
 * biip_rotate_activation, kernels/dispatch.h:229-230, 320-321). Unlike the
 * reference, "ref" is rejected: this library has no CPU path. */
int tqhip_set_ops_impl_by_name(const char *name);
const char *tqhip_ops_impl_name(void);
void tqhip_biip_rotate_activation(const float *x, float *y, int dim, const float *scale, const float *sign,
                                  int block_size);
void tqhip_dispatch_matvec_i4(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size);
void tqhip_dispatch_matvec_pair_i4(const uint8_t *w1, const uint8_t *w2, const float *x, float *y1, float *y2,
                                   int out_dim, int in_dim, int group_size);
void tqhip_dispatch_matvec_qkv_i4(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv, const float *x,
                                  float *yq, float *yk, float *yv, int q_dim, int kv_dim, int in_dim, int group_size);
void tqhip_dispatch_matvec_vq2(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim);
void tqhip_dispatch_matmul_i4(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size);
void tqhip_dispatch_matmul_vq2(const uint8_t *w, const float *x, float *y, int M, int K, int N);

/* ---- 4. byte accounting (runtime/tiny_format.h:73-78, 100-103) --------- */

size_t tqhip_i4_row_bytes(int in_dim, int group_size);
size_t tqhip_vq2_tensor_bytes(int rows, int cols);

/* ---- 5. device plumbing for hosts without a HIP toolchain (tests, bench) */

int tqhip_device_count(void);
int tqhip_device_name(char *buf, int len);
void *tqhip_malloc(size_t bytes);                 /* NULL on failure */
int tqhip_free(void *p);
int tqhip_memcpy_h2d(void *dst, const void *src, size_t bytes);
int tqhip_memcpy_d2h(void *dst, const void *src, size_t bytes);
int tqhip_memcpy_d2d(void *dst, const void *src, size_t bytes);
int tqhip_memset(void *dst, int value, size_t bytes);
int tqhip_synchronize(void);
void *tqhip_stream_create(void);                  /* default priority */
int tqhip_stream_destroy(void *stream);
int tqhip_stream_synchronize(void *stream);
void *tqhip_event_create(void);
int tqhip_event_destroy(void *event);
int tqhip_event_record(void *event, void *stream);
int tqhip_event_elapsed_ms(void *start, void *stop, float *ms);

/* A list of device-pointer calls run back to back on one stream, `repeats`
 * times; used to time a whole decode step with one host call. */
typedef struct tqhip_op {
    int kind;                 /* TQHIP_OP_* */
    const void *w;
    const float *x;
    float *y;
    int out_dim, in_dim, n, group_size;
    const void *w2, *w3;      /* PAIR: w2 / y2; QKV: k = (w2, y2), v = (w3, y3); BIIP: scale, sign */
    float *y2, *y3;
    int out_dim2;             /* QKV: kv_dim (out_dim is q_dim) */
} tqhip_op;
#define TQHIP_OP_I4_MATVEC 1
#define TQHIP_OP_VQ2_MATVEC 2
#define TQHIP_OP_I4_MATMUL 3
#define TQHIP_OP_I4_PAIR 4
#define TQHIP_OP_I4_QKV 5
#define TQHIP_OP_BIIP_ROTATE 6   /* x -> y, in_dim = dim, group_size = block_size, w2 = scale (or NULL), w3 = sign */
#define TQHIP_OP_I4_SET 7        /* w = const tqhip_i4_mat * (n matrices, read when the op runs or is captured), group_size */
#define TQHIP_OP_VQ2_SET 8       /* w = const tqhip_i4_mat * (n VQ2 matrices, read when the op runs or is captured) */
int tqhip_run_ops(const tqhip_op *ops, int n_ops, int repeats, void *stream);
/* As tqhip_run_ops, with a HIP event pair around every call; op_ms[i] gets the
 * mean event-to-event time of call i over the repeats (kernel duration as the
 * stream sees it). */
int tqhip_run_ops_timed(const tqhip_op *ops, int n_ops, int repeats, void *stream, float *op_ms);
/* The op list captured into a HIP graph on `stream` (a created stream, not the
 * null stream) after one eager pass over it, for replay by
 * tqhip_ops_graph_launch. Replays read the buffers the ops name at replay time.
 * The graph owns its scratch (allocated by the eager pass, freed by destroy), so
 * later calls on any stream cannot disturb a replay, and a replay may go to any
 * stream; replays of one graph are ordered among themselves (HIP orders the
 * launches of one executable graph), and destroy waits for the device before
 * freeing the scratch. No counterpart in the reference, whose runtime calls the
 * registry functions one by one: this is for device-resident decode loops,
 * where it cuts the per-kernel launch cost (about 2.8 -> 1.6 us on MI355X). */
int tqhip_ops_graph_create(const tqhip_op *ops, int n_ops, void *stream, void **graph_out);
int tqhip_ops_graph_launch(void *graph, void *stream);
int tqhip_ops_graph_destroy(void *graph);

/* ---- 5b. .tqwen weight files ---------------------------------------------
 * Replaces ModelFile::load (runtime/model_loader.h:228, runtime/model_loader.cpp:267-784)
 * for the files this library serves: format versions 1..3, file dtype f32 / f16 / i4 / VQ2,
 * model types Qwen2 (0) and Qwen3.5 (1). Such a file is accepted exactly when the reference
 * accepts it, with the reference's first failing check as the message (validation stages 1,
 * 2, 4, 4b, 5, 5b). GPTQ-int4 files and the MoE model types (2, 3) are rejected with
 * TQHIP_EFILE. Only the header and the tensor table are read by inspect; upload streams the
 * data region into one HBM allocation, where every tensor keeps its file offset
 * (device = base + offset - data_offset, 64-byte aligned), so the i4 / VQ2 tensors feed the
 * _dev entry points as they are. */
typedef struct tqhip_tensor_info {
    char name[65];            /* NUL-terminated (the file pads names to 64 bytes) */
    int dtype;                /* 0 f32, 1 f16, 3 i4, 4 VQ2 (runtime/tiny_format.h:197-205) */
    int ndim;
    uint64_t shape[4];        /* shape[ndim..3] = 0; i4 / VQ2 are [out_dim, in_dim] */
    uint64_t offset, nbytes;  /* absolute file offset and byte size of the payload */
    const void *device;       /* HBM address after tqhip_model_upload, else NULL */
} tqhip_tensor_info;
/* Model configuration from the header (ModelConfig, runtime/model_loader.h:44-100). */
typedef struct tqhip_model_config {
    int n_layers, hidden_size, intermediate_size, n_heads, n_kv_heads, head_dim, vocab_size, max_seq_len;
    int tied_embeddings;
    float rms_norm_eps, rope_theta;
    int model_type;           /* 0 Qwen2 (also every v1 file), 1 Qwen3.5 */
    int quant_group_size;     /* 0 in v1 files and unquantized files */
    int file_dtype;           /* header dtype: 0 f32, 1 f16, 3 i4, 4 VQ2 */
} tqhip_model_config;
/* Reads and validates `path`; *model gets a handle (TQHIP_OK) or NULL (TQHIP_EFILE, with
 * the reason in err when err_len > 0). Needs no GPU. */
int tqhip_model_inspect(const char *path, void **model, char *err, int err_len);
/* The same for a whole file already in host memory (ModelFile::base(), file_bytes(),
 * runtime/model_loader.h:262-268), as a caller holding a loaded ModelFile has it. The image
 * must stay valid until tqhip_model_upload returns. */
int tqhip_model_inspect_memory(const void *image, uint64_t bytes, void **model, char *err, int err_len);
int tqhip_model_config_get(const void *model, tqhip_model_config *config);
/* Copies the data region to HBM on the current device (once; later calls return TQHIP_OK).
 * TQHIP_EFILE if the file's size changed since inspect, TQHIP_EHIP on a HIP failure. */
int tqhip_model_upload(void *model);
int tqhip_model_tensor_count(const void *model);
int tqhip_model_tensor_at(const void *model, int index, tqhip_tensor_info *info);  /* file order */
/* ModelFile::get (runtime/model_loader.h:298, runtime/model_loader.cpp:793-796): TQHIP_OK, or TQHIP_EBADSHAPE when absent. */
int tqhip_model_find(const void *model, const char *name, tqhip_tensor_info *info);
/* Header fields a caller needs to drive the kernels (ModelConfig, runtime/model_loader.h:44-100). */
int tqhip_model_quant_group_size(const void *model);  /* 0 in v1 files and unquantized files */
int tqhip_model_file_dtype(const void *model);
int tqhip_model_type(const void *model);               /* 0 for v1 files */
void tqhip_model_free(void *model);                   /* frees the HBM copy too */

/* ---- 5c. device-resident decode engine -----------------------------------
 * The gpu_decode boundary (GpuDecodeCreateFn / StepFn / ResetFn / DestroyFn / LogitsFn,
 * kernels/dispatch.h:337-378; the reference's engine is kernels/cuda/gpu_engine.cu, which
 * serves f32 / f16 files). This engine serves dense i4 and VQ2 files (model type 0: Qwen2.x
 * with q/k/v biases, Qwen3 dense with q/k norms; VQ2 files with fp16 or fp32 vectors and a
 * compact-i4 or VQ2 lm_head; BiIP rotations where the file has them): weights as uploaded by
 * tqhip_model_upload, an
 * fp32 KV cache of max_seq_len positions and all activations in HBM, one HIP-graph replay
 * per step; only the token id and the next token cross PCIe.
 *
 * create: max_seq_len <= 0 takes the model's; above it, TQHIP_EBADSHAPE. A missing tensor, a
 * wrong shape or an unsupported file gives TQHIP_EFILE; the message is in err. Uploads the
 * model if it is not yet uploaded; the model must outlive the engine.
 * step: QwenModel::forward_token (runtime/qwen_forward_token.cpp:83) at position
 * seq_len: returns the argmax token of the logits, or TQHIP_EBADSHAPE for a token outside
 * [0, vocab) or a full cache (the reference aborts there), TQHIP_ELAUNCH on a HIP failure.
 * logits: device pointer to the last step's vocab_size logits (valid until destroy).
 *
 * Engines of i4 files whose projections the set kernel takes (group size 64, no rotations) run
 * each layer's residual adds, RMSNorms and SwiGLU inside its projection launches ("fused"),
 * and, with TQHIP_DECODE_FLOW=1 in the environment at create, run a step as one cooperative
 * launch of the whole layer stack whose phases wait for each other's outputs through tagged
 * vectors in HBM, then the lm_head and the argmax ("flow"; the default is the graph, which is
 * as fast or faster on MI355X). The flow step gives the graph step's logits bit for bit; if
 * one of its waits runs out (100 ms), the engine reports it on stderr, runs that token through
 * the graph and keeps to the graph. */
int tqhip_decode_create(void *model, int max_seq_len, char *err, int err_len, void **engine);
int tqhip_decode_step(void *engine, int token_id);
void tqhip_decode_reset(void *engine);      /* back to position 0 (KvCache::reset) */
void tqhip_decode_destroy(void *engine);
const float *tqhip_decode_logits(const void *engine);
int tqhip_decode_seq_len(const void *engine);
/* How the engine runs a step (no counterpart in the reference): TQHIP_DECODE_FUSED |
 * TQHIP_DECODE_FLOW | TQHIP_DECODE_EAGER bits, -1 for a null engine. */
#define TQHIP_DECODE_FUSED 1
#define TQHIP_DECODE_FLOW 2
#define TQHIP_DECODE_EAGER 4
int tqhip_decode_mode(const void *engine);

/* ---- 6. synthetic inputs (portable generator, identical on every host) -- */

uint64_t tq_synth_seed(uint64_t base, int layer, const char *name);
void tq_synth_i4(uint8_t *w, int out_dim, int in_dim, int group_size, uint64_t seed, float scale_lo,
                 float scale_hi, float zero_lo, float zero_hi);
void tq_synth_normal(float *x, long long n, uint64_t seed, float mean, float stddev);
void tq_synth_vq2(uint8_t *w, int out_dim, int in_dim, uint64_t seed, float cb_std);
uint16_t tq_f32_to_f16(float f);

#ifdef __cplusplus
}
#endif

#endif /* TQHIP_H */
