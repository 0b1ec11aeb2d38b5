/*
 * libecpu for MI355X (gfx950): the C ABI of piLM's native library, served by
 * HIP kernels that run on the GPU.
 *
 * Every declaration keeps the name, argument order, struct layout and return
 * codes of the piLM interface it replaces (cited as path:line in the piLM
 * repository), so src/abi/bindings.py can load this library unchanged through
 * PILM_ECPU_LIB.  What changes is where the data lives:
 *
 *   - Matrix/vector pointers passed to ekernel_* are device (HBM) pointers.
 *     A pointer that is not device memory, or a buffer that is smaller than
 *     the shape in the descriptor implies, is rejected with ECPU_ERR_PARAM and
 *     a message in ecpu_last_error(); nothing is launched.
 *   - Kernels are enqueued on the library's current stream (the null stream
 *     unless ecpu_hip_set_stream() chose another) and the call returns without
 *     waiting.  Work queued on that stream afterwards is ordered after it;
 *     the device vtable's synchronize() makes results visible to the host.
 *   - The `isa` argument is accepted and ignored, as in the reference.
 *
 * Numerics: for M < 64 activation rows the linear kernels reproduce the
 * reference CPU kernels' summation order exactly (8 fp32 FMA lanes for int8
 * weights, 2x8 lanes per 16-element chunk for int4, fresh per-group dots
 * folded with one FMA per group), so their outputs are bit-identical to the
 * reference for every shape; so are the fused SwiGLU and argmax entries.
 * For M >= 64 (environment PILM_HIP_MFMA_MIN_M, default 64; 0 disables) the
 * linears run on the matrix cores with fp16 operands and fp32 accumulation:
 * outputs within 1e-2 of the reference per output row.
 */
#ifndef PILM_ECPU_HIP_H
#define PILM_ECPU_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- ecpu_base.h:11-16, 18-26 ------------------------------------------ */
#define ECPU_OK              0
#define ECPU_ERR_PARAM     (-1)
#define ECPU_ERR_MEM       (-2)
#define ECPU_ERR_DEVICE    (-3)  /* a HIP runtime call failed */
#define ECPU_ERR_KERNEL    (-4)
#define ECPU_ERR_UNSUPPORTED (-5)

typedef enum {
    ECPU_PRECISION_F32 = 0,
    ECPU_PRECISION_F16 = 1,
    ECPU_PRECISION_BF16 = 2,
    ECPU_PRECISION_F8_E4M3 = 3,
    ECPU_PRECISION_F8_E5M2 = 4,
    ECPU_PRECISION_I8 = 5,
    ECPU_PRECISION_I4 = 6,
} ecpu_precision_t;

/* ---- device/api.h:11-46: device vtable, gains EDEV_HIP ----------------- */
typedef enum {
    EDEV_ECPU = 0,   /* host memory (posix_memalign), as in the reference   */
    EDEV_CUDA = 1,   /* reserved slot kept for enum compatibility; init -1  */
    EDEV_HIP = 2,    /* MI355X HBM: hipMalloc / hipMemcpy / hipDeviceSynchronize */
    EDEV_COUNT
} edevice_t;

typedef enum {
    EDEV_CAP_NONE = 0,
    EDEV_CAP_F16 = 1 << 0,
    EDEV_CAP_BF16 = 1 << 1,
    EDEV_CAP_FP8 = 1 << 2,
    EDEV_CAP_INT8_AMX = 1 << 3,
    EDEV_CAP_AVX512 = 1 << 4,
    EDEV_CAP_AVX2 = 1 << 5,
    EDEV_CAP_NEON = 1 << 6,
    EDEV_CAP_SVE = 1 << 7,
    EDEV_CAP_NUMA = 1 << 8,
    EDEV_CAP_UNIFIED_MEM = 1 << 9,
    EDEV_CAP_MFMA = 1 << 10,     /* new: CDNA matrix cores */
} edevice_caps_t;

typedef struct edevice_vtable {
    const char *name;
    edevice_t id;
    uint64_t caps;
    void *(*alloc)(size_t bytes, size_t alignment);
    void (*free)(void *ptr);
    void (*memcpy_h2d)(void *dst, const void *src, size_t n);
    void (*memcpy_d2h)(void *dst, const void *src, size_t n);
    void (*memcpy_d2d)(void *dst, const void *src, size_t n);
    int (*synchronize)(void);
    size_t (*mem_total)(void);
    size_t (*mem_free)(void);
    int (*init)(void);
    int (*shutdown)(void);
} edevice_vtable_t;

const edevice_vtable_t *edevice_get(edevice_t dev);                       /* device/api.h:41 */
int edevice_register(edevice_t dev, const edevice_vtable_t *vtable);      /* device/api.h:42 */
int edevice_set_active(edevice_t dev);                                    /* device/api.h:43 */
const edevice_vtable_t *edevice_active(void);                             /* device/api.h:44 */
int edevice_init_all(void);                                               /* device/api.h:45 */
void edevice_shutdown_all(void);                                          /* device/api.h:46 */

/* ---- ecpu.h:23-39: library lifecycle ----------------------------------- */
typedef struct {
    int n_threads;
    int numa_policy;
    int disable_amx;
    int disable_avx512;
    size_t eram_budget_bytes;
    size_t kv_cache_budget_bytes;
    edevice_t device_type;        /* default EDEV_HIP in this library */
} ecpu_config_t;

ecpu_config_t ecpu_config_default(void);                                  /* ecpu.h:33 */
int ecpu_init(const ecpu_config_t *config);                               /* ecpu.h:35 */
void ecpu_shutdown(void);                                                 /* ecpu.h:36 */
int ecpu_is_initialized(void);                                            /* ecpu.h:37 */
const char *ecpu_version(void);                                           /* ecpu.h:38 */
const char *ecpu_last_error(void);                                        /* ecpu.h:39 */

/* ---- kernel/api.h:14-24: ISA enum, gains the GPU target ---------------- */
typedef enum {
    EKERNEL_ISA_SCALAR = 0,
    EKERNEL_ISA_AVX2 = 1,
    EKERNEL_ISA_AVX512 = 2,
    EKERNEL_ISA_AMX = 3,
    EKERNEL_ISA_NEON = 4,
    EKERNEL_ISA_SVE = 5,
    EKERNEL_ISA_GFX950 = 6,
} ekernel_isa_t;

ekernel_isa_t ekernel_detect_isa(void);                                   /* kernel/api.h:23 */
const char *ekernel_isa_name(ekernel_isa_t isa);                          /* kernel/api.h:24 */

/* ---- kernel/api.h:26-38: f32 GEMM (required by bindings.py:_configure) -- */
typedef struct {
    size_t M, N, K;
    ecpu_precision_t a_prec;
    ecpu_precision_t b_prec;
    ecpu_precision_t out_prec;
    int transpose_a;
    int transpose_b;
} ekernel_gemm_desc_t;

int ekernel_gemm(const ekernel_gemm_desc_t *desc, const void *A, const void *B, void *C,
                 ekernel_isa_t isa);                                      /* kernel/api.h:35-38 */

/* ---- kernel/api.h:40-119: the quantized matrix-product path ------------ */
typedef struct {
    size_t M, N, K;
} ekernel_linear_w8a32_desc_t;

/* C[m,n] = scales[n] * sum_k A[m,k] * W[n,k]; A fp32 [M,K], W int8 [N,K],
 * scales fp32 [N], C fp32 [M,N].                          kernel/api.h:52-57 */
int ekernel_linear_w8a32(const ekernel_linear_w8a32_desc_t *desc, const float *A, const int8_t *W,
                         const float *scales, float *C, ekernel_isa_t isa);

/* As above with bf16 A and bf16 (round-to-nearest-even) C.   kernel/api.h:59-64 */
int ekernel_linear_w8a16_bf16(const ekernel_linear_w8a32_desc_t *desc, const uint16_t *A,
                              const int8_t *W, const float *scales, uint16_t *C, ekernel_isa_t isa);

/* Packed int4 W [N, ceil(K/2)] (low nibble = even k, two's complement),
 * per-row fp32 scales [N].                                 kernel/api.h:100-105 */
int ekernel_linear_w4a16_bf16(const ekernel_linear_w8a32_desc_t *desc, const uint16_t *A,
                              const uint8_t *W, const float *scales, uint16_t *C, ekernel_isa_t isa);

/* Packed int4 W with fp32 scales [N, ceil(K/32)] / [N, ceil(K/128)].
 *                                                          kernel/api.h:107-119 */
int ekernel_linear_w4a16g32_bf16(const ekernel_linear_w8a32_desc_t *desc, const uint16_t *A,
                                 const uint8_t *W, const float *scales, uint16_t *C,
                                 ekernel_isa_t isa);
int ekernel_linear_w4a16g128_bf16(const ekernel_linear_w8a32_desc_t *desc, const uint16_t *A,
                                  const uint8_t *W, const float *scales, uint16_t *C,
                                  ekernel_isa_t isa);

/* ---- kernel/api.h:195-198: bf16 SwiGLU (required by _configure) -------- */
/* out[i] = bf16(silu(g) * u), silu(g) = g / (1 + expf(-g)); expf as the
 * reference's C library evaluates it, so outputs are bit-identical. */
int ekernel_swiglu_bf16(const uint16_t *gate, const uint16_t *up, uint16_t *out, size_t n);

/* ---- fused epilogues ---------------------------------------------------- */

/* Greedy decode's lm_head: argmax over n of bf16(scales[n] * A[0,:].W[n,:])
 * for one activation row (M must be 1, N and K nonzero, else
 * ECPU_ERR_UNSUPPORTED); ties and +-0 go to the lowest index, NaN never wins,
 * (-inf, 0) when no value exceeds -inf.  out_index / out_value may each be
 * host memory -- the reference binding's ctypes byref; the call then waits
 * for the result -- or device memory, written by the kernel without waiting.
 *                                          kernel/api.h:66-72, kernels.c:658-737 */
int ekernel_linear_w8a16_bf16_argmax(const ekernel_linear_w8a32_desc_t *desc, const uint16_t *A,
                                     const int8_t *W, const float *scales, size_t *out_index,
                                     float *out_value, ekernel_isa_t isa);

/* The same result with no allocation at all: no counterpart in the reference;
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Its
 * intermediates (the bf16 logits, per-workgroup partials, result, ticket)
 * live in a file-scope device array of about 0.5 MB that each GPU keeps until
 * the process ends, so N is limited to 262144 (larger N: ECPU_ERR_UNSUPPORTED).
 * Calls that overlap in time on one GPU share that array and race. */
int ekernel_linear_w8a16_bf16_argmax_noalloc(const ekernel_linear_w8a32_desc_t *desc, const uint16_t *A,
                                             const int8_t *W, const float *scales, size_t *out_index,
                                             float *out_value, ekernel_isa_t isa);

/*                                                          kernel/api.h:44-50 */
typedef struct {
    size_t M;
    size_t hidden_size;
    size_t intermediate_size;
    size_t gate_up_in_features;
    size_t down_in_features;
} ekernel_w4a16_swiglu_desc_t;

/* The W4 SwiGLU MLP of one token (M must be 1 and down_in_features equal to
 * intermediate_size, else ECPU_ERR_UNSUPPORTED): gate_up_W is packed int4
 * [2I, ceil(K/2)] with per-row scales [2I] (gate rows first), down_W is
 * [H, ceil(I/2)] with scales [H]; C[h] = bf16(down_scales[h] * hidden.down_W[h])
 * with hidden[i] = bf16(silu(g_i) * u_i), g_i and u_i the bf16 outputs of gate
 * row i and up row I+i.  The hidden row lives in a per-device scratch buffer.
 *                                        kernel/api.h:203-214, kernels.c:1598-1735 */
int ekernel_swiglu_w4a16_bf16(const ekernel_w4a16_swiglu_desc_t *desc, const uint16_t *A,
                              const uint8_t *gate_up_W, const float *gate_up_scales,
                              const uint8_t *down_W, const float *down_scales, uint16_t *C,
                              ekernel_isa_t isa);

/* ---- eram.h:12-41: weight residency ------------------------------------ */
typedef struct eram_buffer eram_buffer_t;

typedef enum {
    ERAM_FLAG_NONE = 0,
    ERAM_FLAG_MMAP = 1 << 0,
    ERAM_FLAG_LOCK = 1 << 1,
    ERAM_FLAG_HUGE_PAGES = 1 << 2,
    ERAM_FLAG_NUMA_LOCAL = 1 << 3,
} eram_flags_t;

/* Allocate through the active device (HBM, 256-byte aligned, with EDEV_HIP
 * active); NULL on failure.                                      eram.h:34-37 */
eram_buffer_t *eram_buffer_alloc(size_t bytes, eram_flags_t flags);
void eram_buffer_free(eram_buffer_t *buf);
void *eram_buffer_data(eram_buffer_t *buf);
size_t eram_buffer_size(eram_buffer_t *buf);

/* Map a file read-only into host memory (the reference maps on Windows only
 * and returns NULL elsewhere; this maps on Linux).               eram.h:39-41 */
eram_buffer_t *eram_mmap(const char *path, eram_flags_t flags);
int eram_munmap(eram_buffer_t *buf);
int eram_advise_random(eram_buffer_t *buf);

/* ---- additions (no counterpart in the reference) ----------------------- */

/* Upload n byte ranges of a file into device memory: range i is bytes
 * [file_offsets[i], file_offsets[i] + bytes[i]) and lands at dst[i] (device
 * pointers, checked like kernel arguments).  The file is read in 16 MB chunks
 * into two pinned staging buffers used in turn, each copied to HBM on the
 * library's copy stream while the next is read; returns after the last copy
 * has completed.  For the quantized-weight bundle and cache loaders: one
 * upload per tensor, no per-call copies afterwards. */
int eram_hip_load_file(const char *path, size_t n, const size_t *file_offsets, const size_t *bytes,
                       void *const *dst);

/* Choose the HIP stream the ekernel_* entry points enqueue on (NULL = the
 * null stream).  Callers that run on another stream (e.g. PyTorch's current
 * stream) set it before calling.  Per process, not per thread. */
int ecpu_hip_set_stream(void *hip_stream);
void *ecpu_hip_get_stream(void);

/* Activation rows from which the linear entry points use the matrix-core
 * GEMM (fp16 operands, within 1e-2 of the reference per output row) instead
 * of the bit-exact kernels.  rows >= 0 sets it for the process (0 = never);
 * rows < 0 returns to PILM_HIP_MFMA_MIN_M (default 64).  A caller that needs
 * the reference's bits at any M -- e.g. a batched MTP verify whose tokens
 * must equal per-sequence verification -- sets it above its M.  Not per
 * thread: calls in flight on other threads see the change. */
int ecpu_hip_set_matrix_core_min_rows(int rows);
int ecpu_hip_matrix_core_min_rows(void);

/* Per-call GPU timing of the linear entry points, the native counterpart of
 * the per-linear stage profiler in src/models/base/linear.py:148-169.
 * Between begin and end every linear call records a HIP event pair on its
 * stream around its kernels.  read() waits for those events and writes one
 * line per kernel family: "<family> <calls> <total_ms> <alg_bytes> <flops>",
 * where alg_bytes counts weights + scales + activations + outputs once. */
int ecpu_hip_profile_begin(void);
int ecpu_hip_profile_end(void);
int ecpu_hip_profile_read(char *buf, size_t len);

/* ---- paged attention on device (no C counterpart: the reference runs this
 * step in torch, src/models/qwen3/attention.py:95-139, over the paged cache
 * of src/runtime/kvcache/physical_kv.py:11-81) ----------------------------- */
typedef struct {
    size_t S;            /* query rows (tokens) of this step */
    size_t n_heads;      /* query heads; head h reads kv head h / (n_heads / n_kv_heads) */
    size_t n_kv_heads;
    size_t head_dim;     /* 64, 128 or 256 */
    size_t cache_len;    /* tokens once this step's S rows are in: positions 0 .. cache_len-1,
                            the new rows at cache_len-S .. cache_len-1 */
    size_t block_size;   /* tokens per cache block */
    size_t num_blocks;   /* blocks in each cache tensor */
    size_t n_block_ids;  /* entries of the block table */
    size_t gate_stride;  /* elements between the gates of consecutive (s, h); 0 = no gate */
} ekernel_paged_attention_desc_t;

/* out[s, h*D + d] = bf16(sum_j p[s,h,j] * V[j, h/rep, d]) (times bf16(sigmoid(gate[s,h,d]))
 * when gate is not NULL), with p the bf16 softmax (fp32) of the bf16 scores
 * bf16(bf16(q[s,h,:] . K[j, h/rep, :]) * (1/sqrt(D))) over positions
 * j <= cache_len - S + s (the causal mask), as attention.py:95-139 computes
 * them.  q [S, H, D], k_new / v_new [S, Hkv, D] (after k_norm / rope), caches
 * [num_blocks, block_size, Hkv, D], all bf16; position j lives in block
 * block_ids[j / block_size], slot j % block_size.  The new rows are written
 * into the caches (attention.py:95-97) and attended from k_new / v_new.
 * k_cache = v_cache = NULL attends over the new rows only (cache_len == S,
 * attention.py:115-116).  Gate (s, h, d) is gate[(s*H + h)*gate_stride + d]
 * (the q_proj output's second half: gate = qg + D, gate_stride = 2D).
 * Outputs within one bf16 ulp of the reference except where a score or
 * weight lands on the other side of a rounding boundary (the fp32 sums and
 * the exp differ in their last bits). */
int ekernel_paged_attention_bf16(const ekernel_paged_attention_desc_t *desc, const uint16_t *q,
                                 const uint16_t *k_new, const uint16_t *v_new, uint16_t *k_cache,
                                 uint16_t *v_cache, const int32_t *block_ids, const uint16_t *gate,
                                 uint16_t *out);

/* ---- one Qwen3 decoder layer's torch steps on device (no C counterpart: the
 * reference runs them in torch on the CPU, src/models/base/layers.py:101-195,
 * src/models/qwen3/attention.py:82-139, src/models/qwen3/model.py:54-70).
 * Each reproduces the reference's torch CPU roundings bit for bit (torch's
 * CPU summation orders, SLEEF's expf_u10, bf16 intermediates); the fixture
 * they are checked against was written with torch's AVX2 kernels and oneDNN
 * off, the reference's measured platform. --------------------------------- */
typedef struct {
    size_t rows;         /* rows of x */
    size_t hidden;       /* elements per row, 32 .. 8192 */
    float eps;           /* GemmaRMSNorm eps (layers.py:138) */
} ekernel_rmsnorm_desc_t;

/* GemmaRMSNorm (layers.py:130-147) of each row, optionally after the residual
 * add of TransformerBlock.forward (model.py:63-69): h = bf16(x + residual)
 * (h = x when residual is NULL), residual_out = h (when not NULL),
 * out = bf16(bf16(weight + 1) * bf16(h * (1 / sqrt(mean(h^2) + eps)))), the
 * mean summed in torch's CPU order.  All bf16 [rows, hidden]; out and
 * residual_out may alias x or residual row for row. */
int ekernel_rmsnorm_gemma_bf16(const ekernel_rmsnorm_desc_t *desc, const uint16_t *x, const uint16_t *residual,
                               const uint16_t *weight, uint16_t *out, uint16_t *residual_out);

typedef struct {
    size_t S;              /* tokens of this step */
    size_t n_heads, n_kv_heads, head_dim;
    size_t rot_dim;        /* rotated leading dims (head_dim * partial_rotary_factor) */
    size_t q_stride;       /* elements between consecutive tokens' rows of qg */
    size_t kv_stride;      /* ... of k and of v */
    size_t pos0;           /* position of the first token (ignored when step is given) */
    size_t max_positions;  /* rows of the cos / sin tables */
    size_t block_size, num_blocks, n_block_ids;
    float eps;             /* q_norm / k_norm eps */
} ekernel_qk_rope_desc_t;

/* FullAttention.forward up to the cache write (attention.py:82-97): per token
 * s and head h, q_out[s, h, :] = rope(GemmaRMSNorm(qg[s, h*2D : h*2D + D])),
 * and per kv head the roped, normalized k[s, kh*D ...] and v[s, kh*D ...]
 * stored at position p = pos0 + s of the paged caches [num_blocks,
 * block_size, n_kv_heads, D] (block block_ids[p / block_size], slot p %
 * block_size).  Rope is apply_rope's (layers.py:150-195) with the fp32
 * tables cos/sin [max_positions, rot_dim/2] the caller builds as
 * _rope_cos_sin does.  step (device int32, may be NULL): step[0] replaces
 * pos0, so a captured graph can advance it. */
int ekernel_qk_norm_rope_bf16(const ekernel_qk_rope_desc_t *desc, const uint16_t *qg, const uint16_t *k,
                              const uint16_t *v, const uint16_t *q_norm_w, const uint16_t *k_norm_w,
                              const float *cos_table, const float *sin_table, const int32_t *step,
                              uint16_t *q_out, uint16_t *k_cache, uint16_t *v_cache, const int32_t *block_ids);

typedef struct {
    size_t S, n_heads, n_kv_heads, head_dim;   /* head_dim 64, 128 or 256 */
    size_t cache_len;      /* positions once this step's S tokens are cached (ignored when step is given) */
    size_t block_size, num_blocks, n_block_ids;
    size_t gate_row_stride;    /* elements between tokens' gates (0 with gate NULL) */
    size_t gate_head_stride;   /* elements between heads' gates */
} ekernel_attention_exact_desc_t;

/* attention.py:99-139 over the paged cache (the step's rows already stored):
 * out[s, h*D + d] = bf16(P.V) * bf16(sigmoid(gate[s*gate_row_stride +
 * h*gate_head_stride + d])) with the bf16 scores bf16(bf16(q.k) * (1/sqrt D)),
 * the causal mask j <= cache_len - S + s, fp32 softmax rounded to bf16, and
 * kv head h / (n_heads / n_kv_heads); every sum in torch's CPU order, so the
 * output is bit-identical to the reference's.  step (device int32, may be
 * NULL): step[1] replaces cache_len (clamped to [S, n_block_ids *
 * block_size]).  Block ids outside [0, num_blocks) are clamped, never read
 * out of bounds.  Up to 64 KB of LDS: (n_heads / n_kv_heads) x n_block_ids x
 * block_size positions of scores. */
int ekernel_attention_exact_bf16(const ekernel_attention_exact_desc_t *desc, const uint16_t *q,
                                 const uint16_t *k_cache, const uint16_t *v_cache, const int32_t *block_ids,
                                 const uint16_t *gate, const int32_t *step, uint16_t *out);

/* Several sequences' rows in one launch (continuous batching: an MTP verify
 * step of every running sequence, prefill chunks of several prompts).  No
 * counterpart in the reference, which runs attention per sequence
 * (src/engine.py:416-545 under src/runtime/scheduler/scheduler.py:70-178);
 * each row's result is bit-identical to the per-sequence call's.  Batch rows
 * 0 .. desc->S - 1 (at most 128) are dealt to n_seqs sequences: sequence i
 * owns rows row0 .. row0 + rows - 1 at positions pos0 .. pos0 + rows - 1 and
 * the block table block_ids[table * n_block_ids ...] (block_ids holds
 * n_tables tables of desc->n_block_ids entries).  Every row must belong to
 * exactly one sequence. */
typedef struct {
    int32_t row0;    /* first batch row of the sequence */
    int32_t rows;    /* its rows in this call */
    int32_t pos0;    /* position of its first row (its cached positions before the call) */
    int32_t table;   /* index of its block table in block_ids */
} ekernel_batch_seq_t;

/* ekernel_qk_norm_rope_bf16 for a batch (desc->S = batch rows; pos0 ignored). */
int ekernel_qk_norm_rope_batch_bf16(const ekernel_qk_rope_desc_t *desc, const ekernel_batch_seq_t *seqs,
                                    size_t n_seqs, size_t n_tables, const uint16_t *qg, const uint16_t *k,
                                    const uint16_t *v, const uint16_t *q_norm_w, const uint16_t *k_norm_w,
                                    const float *cos_table, const float *sin_table, uint16_t *q_out,
                                    uint16_t *k_cache, uint16_t *v_cache, const int32_t *block_ids);

/* ekernel_attention_exact_bf16 for a batch (desc->S = batch rows; cache_len
 * ignored: each sequence's is pos0 + rows). */
int ekernel_attention_exact_batch_bf16(const ekernel_attention_exact_desc_t *desc, const ekernel_batch_seq_t *seqs,
                                       size_t n_seqs, size_t n_tables, const uint16_t *q, const uint16_t *k_cache,
                                       const uint16_t *v_cache, const int32_t *block_ids, const uint16_t *gate,
                                       uint16_t *out);

typedef struct {
    size_t rows;      /* activation rows: 1 (one decode token) */
    size_t N;         /* rows of W (with swiglu: gate rows then as many up rows) */
    size_t K;         /* hidden size, a multiple of 256 up to 16384 */
    float eps;        /* GemmaRMSNorm eps */
    int swiglu;       /* 1: out[i] = bf16(bf16(silu(gate_i)) * up_i), N / 2 outputs */
} ekernel_norm_linear_desc_t;

/* The residual add + GemmaRMSNorm before a Linear of TransformerBlock
 * (model.py:63-69: input_layernorm before q/k/v, post_attention_layernorm
 * before gate/up) and that W4A16 g128 Linear, for one token in one launch:
 * h = bf16(x + residual) (x when residual is NULL), residual_out = h (when
 * not NULL), a = GemmaRMSNorm(h) as ekernel_rmsnorm_gemma_bf16 computes it,
 * out = a @ W^T as ekernel_linear_w4a16g128_bf16 computes it; with swiglu
 * the SwiGLU product F.silu(gate) * up of the two halves of W
 * (layers.py:188-193) as ekernel_silu_mul_bf16 computes it.  Bit-identical
 * to those calls in sequence.  All pointers 16-byte aligned (scales 4);
 * residual_out and out must not overlap x or residual.  No counterpart in
 * the reference, which runs these steps one after another. */
int ekernel_rmsnorm_linear_w4a16g128_bf16(const ekernel_norm_linear_desc_t *desc, const uint16_t *x,
                                          const uint16_t *residual, const uint16_t *norm_weight,
                                          uint16_t *residual_out, const uint8_t *W, const float *scales,
                                          uint16_t *out);

/* One decode row (S = 1) of FullAttention.forward (attention.py:82-139) in
 * one launch: ekernel_qk_norm_rope_bf16 followed by
 * ekernel_attention_exact_bf16 with the gate inside qg (gate_row_stride
 * n_heads*2*head_dim, gate_head_stride 2*head_dim), bit-identical to them,
 * the roped q kept on chip.  desc as for ekernel_qk_norm_rope_bf16 with
 * S = 1; the cache holds pos0 + 1 positions after the call (step: step[0]
 * the position, step[1] the cached length, as the two calls read them).
 * head_dim 64 or 128, 1, 2 or 4 q heads per kv head, the visible value
 * rows staged in LDS in passes.  out [n_heads * head_dim] bf16. */
int ekernel_decode_attention_bf16(const ekernel_qk_rope_desc_t *desc, const uint16_t *qg, const uint16_t *k,
                                  const uint16_t *v, const uint16_t *q_norm_w, const uint16_t *k_norm_w,
                                  const float *cos_table, const float *sin_table, const int32_t *step,
                                  uint16_t *k_cache, uint16_t *v_cache, const int32_t *block_ids, uint16_t *out);

/* out[m, i] = bf16(bf16(silu(gate[m*in_stride + i])) * up[m*in_stride + i])
 * (F.silu(gate(x)) * up(x), layers.py:188-193), m < rows, i < n. */
int ekernel_silu_mul_bf16(const uint16_t *gate, const uint16_t *up, size_t rows, size_t n, size_t in_stride,
                          uint16_t *out);

/* Greedy decode step on device: id = argmax of the bf16 logits[n] (the first
 * index of the largest value, as torch.argmax picks it for finite logits,
 * src/engine.py:551); then tokens[state[2]] = id (while state[2] <
 * max_tokens), state[2] += 1, *next_id = id, state[0] = state[1],
 * state[1] += 1 (state = {pos0, cache_len, count}, the decode position
 * advancing for the next step). */
int ekernel_greedy_step_bf16(const uint16_t *logits, size_t n, int32_t *state, int32_t *tokens, size_t max_tokens,
                             int64_t *next_id);

#ifdef __cplusplus
}
#endif

#endif /* PILM_ECPU_HIP_H */
