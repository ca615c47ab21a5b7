/*
 * nomas_moe.h -- C ABI of the MI355X (gfx950) top-k MoE feed-forward block.
 *
 * Drop-in for hy-nomas-rs `MoeLayer` (nomas-core/src/modules/moe.rs).  Every
 * entry point below names the reference interface it replaces.  Plain
 * pointers and sizes only; a Rust `extern "C"` block binds it 1:1.
 *
 * Conventions
 *  - Every function returning `int` returns NOMAS_OK (0) or a NOMAS_ERR_* code;
 *    the message of the last failure on the calling thread is available from
 *    nomas_moe_last_error().  These map onto the reference's error variants
 *    (nomas-core/src/error.rs:7-46): INVALID_CONFIG -> Error::InvalidConfig,
 *    WEIGHT_KEY -> Error::WeightKey, everything else -> Error::Candle /
 *    Error::Msg.  A checkpoint that cannot be read or parsed (IO) is the
 *    reference's Error::Msg("loading <path>: <reason>"): load_dit maps every
 *    load failure to that message (weights.rs:112-115), and NOMAS_ERR_IO
 *    carries the same text.  No entry point lets a C++ exception or an abort
 *    escape: failures are always a returned status.
 *  - Tensors are row-major.  A forward input of any rank >= 2 with last dim D
 *    is passed as `rows` = product of the leading dims, exactly as Lin::fwd
 *    folds leading dims (nomas-core/src/modules/mod.rs:132-134).
 *  - Weights use the reference's (out, in) layout with experts concatenated:
 *    router (E, D); gate/up (E, H, D) + bias (E, H); down (E, D, H) + bias (E, D).
 *  - dtype codes follow nomas-core/src/config.rs:30-39 (DataType).
 *  - A handle owns its device weights and workspace.  Forwards on one handle
 *    are ordered: one issued on a different stream than the previous one
 *    waits (on the device) for it to finish, since they share the workspace.
 *    A handle must not be called from several host threads at once; use one
 *    handle per thread for concurrency.
 */
#ifndef NOMAS_MOE_H
#define NOMAS_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum nomas_status {
    NOMAS_OK = 0,
    NOMAS_ERR_INVALID_CONFIG = 1,   /* config.rs:394-399 / shapes unsupported      */
    NOMAS_ERR_INVALID_ARGUMENT = 2, /* null or misaligned pointer, bad row count   */
    NOMAS_ERR_WEIGHT_KEY = 3,       /* weights.rs:117-127 missing / misshaped key  */
    NOMAS_ERR_IO = 4,               /* checkpoint unreadable or malformed          */
    NOMAS_ERR_HIP = 5,              /* a HIP runtime call failed                   */
    NOMAS_ERR_OUT_OF_MEMORY = 6,    /* device or host allocation failed            */
    NOMAS_ERR_STATE = 7,            /* e.g. routing read back before any forward   */
    NOMAS_ERR_INTERNAL = 8          /* an unexpected failure inside the library    */
};

/* DataType (config.rs:30-39). */
enum nomas_dtype { NOMAS_F32 = 0, NOMAS_BF16 = 1, NOMAS_F16 = 2 };

/* MoeConfig (config.rs:202-213), field for field. */
typedef struct nomas_moe_config {
    int64_t experts;     /* number of experts                                   */
    int64_t top_k;       /* experts activated per token                         */
    double shared_dense; /* coefficient of the additive shared dense FFN (moe.rs:103-106) */
    uint64_t seed;       /* carried for parity; unused, as in the reference     */
} nomas_moe_config;

typedef struct nomas_moe nomas_moe_t;

/* NomasConfig::validate's MoE clause (config.rs:394-399): 1 <= top_k <= experts. */
int nomas_moe_config_validate(const nomas_moe_config *cfg);

/* MoeLayer::from_source with Weights::Random (moe.rs:26-62, mod.rs:38-45,80-95):
 * router and experts drawn by xavier(path_seed(seed, "{path}.router" /
 * "{path}.experts.{e}.{gate,up,down}" / "{path}.dense.*")), zero biases,
 * rounded to `dtype`.  `device` is the HIP device ordinal. */
int nomas_moe_from_random(const nomas_moe_config *cfg, const char *path, int64_t dim,
                          int64_t hidden, int dtype, uint64_t seed, int device,
                          nomas_moe_t **out);

/* MoeLayer::from_source with Weights::Loaded (moe.rs:26-62, mod.rs:69-77,
 * weights.rs:105-145): reads `{path}.router.weight`,
 * `{path}.experts.{e}.{gate,up,down}.{weight,bias}` and, when shared_dense > 0,
 * `{path}.dense.*` from the given safetensors files (later files override
 * earlier ones), casting every tensor to `dtype` (weights.rs:129-133). */
int nomas_moe_from_safetensors(const nomas_moe_config *cfg, const char *const *files,
                               int64_t n_files, const char *path, int64_t dim, int64_t hidden,
                               int dtype, int device, nomas_moe_t **out);

/* MoeLayer from host arrays already in `dtype` (the tensors a VarBuilder would
 * hand to Lin::load, mod.rs:69-77).  Bias pointers may be NULL (zero bias);
 * the dense_* group is read only when cfg->shared_dense > 0. */
int nomas_moe_from_host(const nomas_moe_config *cfg, int64_t dim, int64_t hidden, int dtype,
                        int device, const void *router_w,
                        const void *gate_w, const void *gate_b,
                        const void *up_w, const void *up_b,
                        const void *down_w, const void *down_b,
                        const void *dense_gate_w, const void *dense_gate_b,
                        const void *dense_up_w, const void *dense_up_b,
                        const void *dense_down_w, const void *dense_down_b,
                        nomas_moe_t **out);

/* MoeLayer::forward (moe.rs:65-109) on device-resident tensors: x and y are
 * (rows, D) in the handle's dtype, 16-byte aligned; `stream` is a
 * hipStream_t (NULL = default stream).  Asynchronous with respect to the host. */
int nomas_moe_forward(nomas_moe_t *h, const void *x, void *y, int64_t rows, void *stream);

/* No counterpart in the reference: nomas_moe_forward for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments and results, but every device buffer of
 * the forward (routing, permuted rows, the SwiGLU intermediate, K-split
 * partials) lives in a static device array of 512 MiB per GPU, held until
 * the process ends: the call allocates nothing.  `rows` beyond what fits (it
 * depends on dim, hidden and top_k; 8,128 rows at dim 3072, hidden 8192,
 * top-2, so one 4,744-row segment of the 8B preset) is
 * NOMAS_ERR_INVALID_ARGUMENT with the limit in the message.  The
 * first call on a device looks up the array's address and clears its
 * counters with a kernel on `stream`.  All such calls on one GPU share the
 * array: calls that overlap on one GPU (different streams, threads or
 * handles) race, and routing() after such a call reads the array: once
 * another no-allocation forward has run on the GPU, routing() on the first
 * handle is NOMAS_ERR_STATE. */
int nomas_moe_forward_noalloc(nomas_moe_t *h, const void *x, void *y, int64_t rows, void *stream);

/* The FFN half of DiTBlock::forward around the MoE (block.rs:96-101), fused
 * into the MoE's own kernels:
 *   h   = modulate(norm2(x), shift, scale)     (norm.rs:55-65, modulate.rs:69-79)
 *   out = x + moe(h) * gate
 * x and out are (rows, D) in the handle's dtype, device-resident, 16-byte
 * aligned (out may alias x); row r belongs to sequence r / seq (rows must be a
 * multiple of seq).  shift, scale and gate are (rows / seq, D) f32 on the
 * device, 16-byte aligned: the AdaLN parameters of the batch (AdaSix::{shift,scale,gate}_mlp,
 * modulate.rs:13-27).  norm_w is norm2's affine gain widened to f32 (D
 * entries) or NULL for RmsNorm::no_affine; eps is norm2's (1e-6 in
 * DiTBlock::from_source, block.rs:56-57).  Rounding to the model dtype happens
 * where the reference's to_dtype casts do (after the norm, after modulate, on
 * the MoE output, on y * gate and on the sum); the row's sum of squares is
 * the reference's serial f32 chain, one rounded add per element in ascending
 * column order (norm.rs:58-65).  For an F32 handle this is the reference's arithmetic;
 * for BF16/F16 the reference's modulate (an F32 tensor times model-dtype
 * parameters) does not type-check in candle, and this entry point defines the
 * block with the f32 parameters above.  The router sees h, so routing()
 * reports h's routing; with shared_dense > 0 the dense branch reads h too.
 * Dense (nomas_ffn_t) handles have no fused block. */
int nomas_moe_forward_block(nomas_moe_t *h, const void *x, void *out, int64_t rows, int64_t seq,
                            const float *norm_w, double eps, const float *shift,
                            const float *scale, const float *gate, void *stream);

/* MoeLayer::forward on host tensors (the candle CPU-tensor case): copies x in,
 * runs the forward, copies y out and synchronises.  Pageable buffers are
 * staged through the handle's pinned buffers (a threaded host copy overlapping
 * the DMA); pinned buffers (hipHostMalloc'd) go straight to DMA.  The device
 * copies of x and y stay with the handle between calls. */
int nomas_moe_forward_host(nomas_moe_t *h, const void *x, void *y, int64_t rows);

/* MoeLayer::n_params (moe.rs:112-114): router + experts, dense excluded. */
int64_t nomas_moe_n_params(const nomas_moe_t *h);

/* Routing of the last forward, read back to host (no reference counterpart:
 * the reference keeps it inside forward, moe.rs:92-95).  idx/w are rows x k
 * with experts in ascending index order, counts has E entries, gap has one
 * entry per row: logit of the k-th selected expert minus the best unselected
 * one (+inf when k == E).  Any pointer may be NULL.  Synchronises.
 * NOMAS_ERR_STATE before any forward, and after a forward that failed (its
 * launches may have overwritten the previous forward's routing). */
int nomas_moe_routing(nomas_moe_t *h, int32_t *idx, float *w, int32_t *counts, float *gap);

/* Dimensions of a handle: dim, hidden, experts, top_k, dtype (any may be NULL). */
int nomas_moe_dims(const nomas_moe_t *h, int64_t *dim, int64_t *hidden, int64_t *experts,
                   int64_t *top_k, int *dtype);

/* Per-stage timing (no reference counterpart; measurement only).  When enabled,
 * each forward's kernels carry HIP events that the runtime stamps at the start
 * of a stage's first kernel and the end of its last, so a stage's time is its
 * kernels' own (no launch gap); a stage without a kernel reads zero.
 * nomas_moe_stage_times returns the mean over the forwards recorded since the
 * last call, in milliseconds: [router, scan, dispatch, gemm_gate_up,
 * gemm_down, combine] ("scan" is part of the dispatch kernel and reads zero).
 * Synchronises. */
int nomas_moe_set_profiling(nomas_moe_t *h, int enable);
int nomas_moe_stage_times(nomas_moe_t *h, float *ms6);

/* Which GEMM path the handle uses: 1 = MFMA grouped GEMM (dim a multiple of
 * 256 and hidden a multiple of 128, any dtype), 0 = general (any shape) path. */
int nomas_moe_uses_mfma(const nomas_moe_t *h);

void nomas_moe_destroy(nomas_moe_t *h);

/* ---- Dense SwiGLU feed-forward ------------------------------------------------
 * FeedForward::SwiGlu (nomas-core/src/modules/mlp.rs:9-59), the FFN of the DiT
 * blocks when the config has no MoE (BlockFfn::Dense, block.rs:14-19,47-53):
 * y = down(silu(gate(x)) * up(x)) with biases.  It runs on the same grouped
 * GEMM kernels as the experts (one expert, no routing); the MoE conventions
 * above apply (errors, dtypes, row folding, stream ordering). */
typedef struct nomas_ffn nomas_ffn_t;

/* FeedForward::from_source with Weights::Random (mlp.rs:18-37, mod.rs:38-45,
 * 80-95): `{path}.gate`, `{path}.up`, `{path}.down`, each a xavier weight from
 * path_seed(seed, key) and a zero bias, cast to `dtype`. */
int nomas_ffn_from_random(const char *path, int64_t dim, int64_t hidden, int dtype,
                          uint64_t seed, int device, nomas_ffn_t **out);

/* FeedForward::from_source with Weights::Loaded over load_dit's cast
 * (mlp.rs:18-37, weights.rs:105-145): reads `{path}.{gate,up,down}.{weight,bias}`
 * from the safetensors files; missing keys are NOMAS_ERR_WEIGHT_KEY with the
 * reference's message. */
int nomas_ffn_from_safetensors(const char *const *files, int64_t n_files, const char *path,
                               int64_t dim, int64_t hidden, int dtype, int device,
                               nomas_ffn_t **out);

/* Lin::load of materialised tensors (mod.rs:69-77): host arrays in the model
 * dtype, reference layout gate/up (H, D) + (H), down (D, H) + (D); biases may
 * be null (zero). */
int nomas_ffn_from_host(int64_t dim, int64_t hidden, int dtype, int device, const void *gate_w,
                        const void *gate_b, const void *up_w, const void *up_b,
                        const void *down_w, const void *down_b, nomas_ffn_t **out);

/* FeedForward::forward (mlp.rs:39-48) on device rows (x, y: rows x D, 16-byte
 * aligned) on `stream`, and on host rows (copied in and out). */
int nomas_ffn_forward(nomas_ffn_t *h, const void *x, void *y, int64_t rows, void *stream);
int nomas_ffn_forward_host(nomas_ffn_t *h, const void *x, void *y, int64_t rows);

/* FeedForward::n_params (mlp.rs:50-58). */
int64_t nomas_ffn_n_params(const nomas_ffn_t *h);

/* No counterpart: per-stage timing ([0, tile table, K-blocked copy of x,
 * gemm_gate_up, gemm_down, 0]) and the GEMM path, as for the MoE handle. */
int nomas_ffn_set_profiling(nomas_ffn_t *h, int enable);
int nomas_ffn_stage_times(nomas_ffn_t *h, float *ms6);
int nomas_ffn_uses_mfma(const nomas_ffn_t *h);

void nomas_ffn_destroy(nomas_ffn_t *h);

/* ---- Block seams on their own ---------------------------------------------------
 * The two expressions of DiTBlock::forward around its FFN (block.rs:96,101),
 * for callers that run the FFN separately (the dense FeedForward of
 * BlockFfn::Dense, block.rs:97-100).  Same conventions as
 * nomas_moe_forward_block: (rows, dim) tensors in `dtype` on the device,
 * 16-byte aligned, dim % 8 == 0, row r in sequence r / seq, f32 (rows / seq,
 * dim) AdaLN parameters and f32 norm gain (16-byte aligned too), asynchronous
 * on `stream` (of the current device). */

/* h = modulate(norm2(x), shift, scale)  (block.rs:96; norm.rs:55-65,
 * modulate.rs:69-79).  norm_w: norm2's gain as f32 or NULL (no_affine).
 * h may alias x. */
int nomas_norm_modulate(int dtype, const void *x, void *h, int64_t rows, int64_t dim, int64_t seq,
                        const float *norm_w, double eps, const float *shift, const float *scale,
                        void *stream);

/* out = x + y * gate  (block.rs:101), y the FFN output; out may alias x or y. */
int nomas_gated_residual(int dtype, const void *x, const void *y, const float *gate, void *out,
                         int64_t rows, int64_t dim, int64_t seq, void *stream);

/* Message of the last failure on this thread ("" if none). */
const char *nomas_moe_last_error(void);

/* Weights::path_seed (mod.rs:47-55): FNV-1a of `path` with the offset basis
 * xor'ed with `seed`. */
uint64_t nomas_path_seed(uint64_t seed, const char *path);

/* deterministic_randn_affine (tensor_utils.rs:123-138): n f32 values of the
 * SplitMix64 + Box-Muller stream `seed`, scaled by std and shifted by mean.
 * Bit-identical to the reference; runs on host threads. */
void nomas_randn_affine(uint64_t seed, double mean, double std, int64_t n, float *out);

/* Host conversion helpers: f32 -> bf16 / f16 bit patterns, round to nearest
 * even (candle's to_dtype, weights.rs:129-133). */
void nomas_f32_to_bf16(const float *in, uint16_t *out, int64_t n);
void nomas_f32_to_f16(const float *in, uint16_t *out, int64_t n);

#ifdef __cplusplus
}
#endif

#endif /* NOMAS_MOE_H */
