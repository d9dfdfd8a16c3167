/* llima_sampler.h -- C ABI of the MI355X logits -> token-selection library
 * (libllima_sampler.so, built for gfx950).
 *
 * Every entry point takes device pointers (any HIP allocation, e.g. a PyTorch
 * ROCm tensor's data_ptr()), plain sizes, a caller-owned workspace and a
 * hipStream_t passed as void* (NULL = the default stream).  Launches are
 * asynchronous on that stream; the return value only reports argument and
 * launch errors.  No entry point allocates memory and no C++ exception
 * crosses this boundary.
 *
 * Workspace contract: a workspace is scratch of at least the size the matching
 * *_workspace_bytes function returns; no state survives a call, so it needs no
 * initialisation and any large-enough buffer may be reused for any shape.  Calls
 * that share one workspace must be ordered (same stream, or synchronised).
 * Each entry point launches a fixed sequence of kernels with no host
 * synchronisation and no memset, so it can be captured in a HIP graph.
 *
 * Reference interfaces replaced (sima-neat/llima, paths relative to that repo).
 * The reference selects tokens on the host CPU through free functions and
 * private LanguageModel members over host-mapped bf16 buffers; these entry
 * points take the same inputs and semantics on device memory:
 *   llima_argmax          <- argmax_bf16              sima_lmm/devkit/cpp/utils.hpp:80-152
 *                            _calc_next_token_id      sima_lmm/devkit/cpp/language_model.cpp:3689-3714
 *                            _argmax_lm_head_row(s)   sima_lmm/devkit/cpp/language_model.cpp:3616-3687
 *                            spec-path argmax         sima_lmm/devkit/cpp/language_model.cpp:1518-1611
 *                            EAGLE3 verify argmax     sima_lmm/devkit/cpp/language_model_eagle3.cpp:486-522
 *                            DFlash proposals         sima_lmm/devkit/cpp/language_model_dflash.cpp:334-349
 *   llima_argmax_splits   <- the same functions over the n{N}_lm_split{i} buffers
 *                            (_prepare_lm_head_logit_views language_model.cpp:3584-3613)
 *   llima_verify_greedy(_splits) <- _argmax_lm_head_rows + resolve_draft_tokens
 *                            sima_lmm/devkit/cpp/language_model.cpp:3636-3687,
 *                            sima_lmm/devkit/cpp/gemma4_mtp_helpers.cpp:81-111
 *   llima_verify_tree     <- tree_decoding gather + evaluate_posterior
 *                            sima_lmm/devkit/cpp/language_model_eagle3.cpp:530-567,
 *                            sima_lmm/devkit/cpp/eagle_helpers.hpp:153-195
 *   llima_sample          <- no reference counterpart: the reference decodes
 *                            greedily only (sima_lmm/devkit/cpp/zmq_server.cpp:39,
 *                            sima_lmm/mole/multimodal.py:89-95); the config
 *                            names follow the HF GenerationConfig fields the
 *                            reference's compiler writes (sima_lmm/model/base.py:554-583).
 *   llima_verify_rejection <- no reference counterpart (the reference verifies
 *                            drafts greedily, eagle_helpers.hpp:153-195); the
 *                            greedy limit equals resolve_draft_tokens.
 *   llima_score_logits    <- score_logits             sima_lmm/devkit/cpp/language_model.cpp:29-62
 *   llima_mtp_masked_argmax <- select_candidate_tokens
 *                            sima_lmm/devkit/cpp/gemma4_mtp_helpers.cpp:113-167,
 *                            _argmax_gemma4_mtp_masked_row
 *                            sima_lmm/devkit/cpp/language_model_gemma4_mtp.cpp:31-97
 *   llima_topk            <- topk<T>                  sima_lmm/devkit/cpp/utils.hpp:216-281
 *   llima_eagle3_tree_*   <- topk_generate's selection steps (topk, logsoftmax,
 *                            cumulative scores, tree mask, position ids,
 *                            retrieve indices, searchsorted)
 *                            sima_lmm/devkit/cpp/language_model_eagle3.cpp:808-1164,
 *                            sima_lmm/devkit/cpp/utils.hpp:283-301,
 *                            sima_lmm/devkit/cpp/eagle_helpers.hpp:197-214
 *   llima_stop_check      <- the decode loop's stop-token check
 *                            sima_lmm/devkit/cpp/language_model.cpp:643-671,
 *                            language_model_dflash.cpp:570-579,
 *                            language_model_gemma4_mtp.cpp:940-956
 *   llima_lm_head_argmax  <- the in-graph LM head + softcap + argmax
 *                            sima_lmm/model/language_part_base.py:171-180,
 *                            sima_lmm/model/model_graph.py:601, 868-870, whose
 *                            int32 the host reads at language_model.cpp:1607-1609
 *   llima_lm_head_pack, llima_lm_head_argmax_packed <- the same, over a weight
 *                            prepacked at load time (no counterpart)
 *   llima_lm_head_score(_packed) <- the LM head followed by score_logits
 *                            (language_model.cpp:29-62), the logits never written
 *   llima_lm_head_verify_greedy(_packed) <- the verification step's LM head +
 *                            _argmax_lm_head_rows + resolve_draft_tokens, no logits
 *   llima_lm_head_verify_tree(_packed) <- the EAGLE3 tree step's LM head + verify
 *                            argmax + tree_decoding + evaluate_posterior, no logits
 */
#ifndef LLIMA_SAMPLER_H
#define LLIMA_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes (the reference raises std::invalid_argument / std::runtime_error
 * for the corresponding conditions, e.g. utils.hpp:86, gemma4_mtp_helpers.cpp:89). */
enum {
    LLIMA_OK = 0,
    LLIMA_E_INVAL = -1,      /* bad argument: size, dtype, config value */
    LLIMA_E_RANGE = -2,      /* id or length out of range */
    LLIMA_E_HIP = -3,        /* the HIP runtime reported an error at launch */
    LLIMA_E_WORKSPACE = -4,  /* workspace missing or too small */
    LLIMA_E_SCRATCH = -5,    /* the call needs more than the static scratch holds */
    LLIMA_E_CAPTURE = -6     /* a first call on a device made under stream capture */
};

enum { LLIMA_F32 = 0, LLIMA_BF16 = 1 };

/* OR'ed into the LM head's logit_dtype together with LLIMA_BF16: out_logits
 * then points to bf16 [B][V] (uint16 bits) and receives each logit as the
 * bf16 value it was rounded to, half the bytes of the fp32 output, which
 * llima_sample reads as LLIMA_BF16 rows.  No counterpart in the reference,
 * whose graphs keep their logits in bf16 (model_graph.py:30-45). */
#define LLIMA_LOGITS_OUT_BF16 0x100

/* A call with B = 0 rows (or sequences) launches nothing and returns LLIMA_OK
 * once its sizes and modes are valid; its per-row buffers may then be null. */

/* argmax modes (NaN and split handling of the reference variants):
 *  SPLIT_FIRST: per split, argmax_bf16 semantics (start at the split's first
 *               value, strict '>': a NaN first value hides its split); splits
 *               merged from (-inf, 0) keeping the greater value, or the lower
 *               index on equal values; an all -inf row gives id 0.  The splits
 *               are split_dim values each (one split when split_dim <= 0: that
 *               is argmax_bf16 itself) or the split buffers of the *_splits
 *               entry points (_argmax_lm_head_row, language_model.cpp:3616-3633).
 *  NEG_INF:     start at -inf, strict '>' over the row: NaN never wins and an
 *               all -inf/NaN row gives id 0 (language_model_eagle3.cpp:486-522).
 *  QUARTERS:    four parts [V*p/4, V*(p+1)/4) merged from (values[0], 0), as
 *               _calc_next_token_id (language_model.cpp:3689-3714).
 *  LOWEST:      start at bf16 lowest() = -3.38953139e38 with index 0, strict
 *               '>' over the row (every split in order): NaN, -inf and values
 *               <= lowest() never win, and such a row gives id 0 (the
 *               speculative path's multi-split scan, language_model.cpp:1556-1575;
 *               its single-split scan is SPLIT_FIRST). */
enum { LLIMA_ARGMAX_SPLIT_FIRST = 0, LLIMA_ARGMAX_NEG_INF = 1, LLIMA_ARGMAX_QUARTERS = 2,
       LLIMA_ARGMAX_LOWEST = 3 };

/* Sampler configuration (host struct).  Scalars apply to every row unless the
 * matching *_rows device pointer (length B) is non-NULL.
 *   temperature        <= 0 (or greedy != 0) selects the argmax of the
 *                      penalised, masked row (lowest index on ties)
 *   top_k              <= 0 or >= V disables.  With top_k_rows given, a scalar
 *                      in (0, V) states that every row's entry is in (0, V):
 *                      the call then skips the finish that can split rows
 *                      without top-k (~1.8 us at 64 x 128256); a row that breaks
 *                      the statement still gets the right token, by the slower
 *                      one-workgroup path.  0 makes no statement.
 *   top_p              >= 1 (or NaN) disables
 *   min_p              <= 0 (or NaN) disables
 *   repetition_penalty 1 disables (HF: score < 0 ? score * p : score / p)
 *   presence_penalty, frequency_penalty  0 disables (OpenAI convention) */
typedef struct llima_sampler_config {
    float temperature;
    int32_t top_k;
    float top_p;
    float min_p;
    float repetition_penalty;
    float presence_penalty;
    float frequency_penalty;
    int32_t greedy;
    const float* temperature_rows;
    const int32_t* top_k_rows;
    const float* top_p_rows;
    const float* min_p_rows;
    const float* repetition_penalty_rows;
    const float* presence_penalty_rows;
    const float* frequency_penalty_rows;
} llima_sampler_config;

/* Greedy selection over B rows of V logits (dtype LLIMA_F32 or LLIMA_BF16, row
 * r at logits + r*row_stride elements).  out_ids[B] receives the index;
 * out_vals[B] (nullable) the selected value as fp32.  The workspace size
 * covers llima_argmax_splits over the same B and total V as well. */
size_t llima_argmax_workspace_bytes(int32_t B, int32_t V, int32_t dtype);
int llima_argmax(const void* logits, int32_t dtype, int32_t B, int32_t V, int64_t row_stride,
                 int32_t split_dim, int32_t mode, int32_t* out_ids, float* out_vals,
                 void* workspace, size_t workspace_bytes, void* stream);

/* Greedy selection over rows held in n_splits (1..16) split buffers, the
 * layout of the reference's n{N}_lm_split{i} LM-head outputs
 * (_prepare_lm_head_logit_views, language_model.cpp:3584-3613): splits[i] (a
 * host array of device pointers) holds vocabulary ids [sum of the widths before
 * i, + split_widths[i]) of every row, row r at splits[i] + r*split_row_strides[i]
 * elements (split_row_strides nullable: the widths).  V = sum of the widths.
 * Modes SPLIT_FIRST (each buffer a split), NEG_INF and LOWEST. */
int llima_argmax_splits(const void* const* splits, const int32_t* split_widths,
                        const int64_t* split_row_strides, int32_t n_splits, int32_t dtype,
                        int32_t B, int32_t mode, int32_t* out_ids, float* out_vals,
                        void* workspace, size_t workspace_bytes, void* stream);

/* Full sampler over B rows: grammar bitmask (nullable, [B][ceil(V/32)] uint32,
 * bit i of word i>>5 LSB-first, 0 = masked), history (nullable, [B][H_max]
 * int32 token ids; ids outside [0, V) are ignored; history_len nullable [B]),
 * repetition -> frequency/presence penalties, temperature, top-k, top-p, min-p,
 * and an inverse-CDF draw with uniforms[B] in [0, 1).
 * out_ids[B]: token id, or -1 when no token is admissible (every value masked
 * or -inf).  out_probs[B] (nullable): the token's probability under the final
 * distribution (1 for greedy rows).  out_keep (nullable, [B][ceil(V/32)]):
 * the final kept set as a bitmask (finite values only). */
size_t llima_sample_workspace_bytes(int32_t B, int32_t V, int32_t dtype);
int llima_sample(const void* logits, int32_t dtype, int32_t B, int32_t V, int64_t row_stride,
                 const int32_t* history, const int32_t* history_len, int32_t H_max,
                 const uint32_t* bitmask, const float* uniforms,
                 const llima_sampler_config* cfg, int32_t* out_ids, float* out_probs,
                 uint32_t* out_keep, void* workspace, size_t workspace_bytes, void* stream);

/* llima_sample without a workspace argument.  No counterpart in the reference:
 * it serves callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops and harnesses that forbid hipMalloc).  The workspace
 * is a static device array of llima_sample_noalloc_max_bytes() (48 MiB) bytes
 * per GPU, allocated when the library is loaded on that GPU and held until the
 * process ends; the call allocates nothing.  Calls whose
 * llima_sample_workspace_bytes(B, V, dtype) exceed it return LLIMA_E_SCRATCH
 * (the workspace is 5 KB per row and 16 KB chunk plus 64 bytes per row:
 * B*(5120*ceil(V/4096) + 64) <= 48 MiB for fp32 rows, with ceil(V/8192) for bf16).
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (different streams, or different host threads without ordering) race.
 * The first call on a device looks the array's address up (once) and must be
 * made outside stream capture: made under capture it launches nothing and
 * returns LLIMA_E_CAPTURE.  Later calls on that device may be captured and
 * replayed.  Results are those of llima_sample on the same inputs. */
size_t llima_sample_noalloc_max_bytes(void);
int llima_sample_noalloc(const void* logits, int32_t dtype, int32_t B, int32_t V,
                         int64_t row_stride, const int32_t* history, const int32_t* history_len,
                         int32_t H_max, const uint32_t* bitmask, const float* uniforms,
                         const llima_sampler_config* cfg, int32_t* out_ids, float* out_probs,
                         uint32_t* out_keep, void* stream);

/* Greedy chain verification of B sequences with D draft tokens each.
 * target_logits: [B][D+1][V]; draft_ids: [B][D].  Each target row's argmax
 * follows split_dim and mode as llima_argmax (SPLIT_FIRST with the head's
 * split_dim is _argmax_lm_head_rows, language_model.cpp:3636-3687).
 * accepted_len[B] = length of the matching prefix; emitted[B][D+1] = accepted
 * drafts, then the target argmax at the first mismatch (or the bonus token),
 * then -1 padding. */
size_t llima_verify_greedy_workspace_bytes(int32_t B, int32_t D, int32_t V, int32_t dtype);
int llima_verify_greedy(const void* target_logits, int32_t dtype, int32_t B, int32_t D,
                        int32_t V, int32_t split_dim, int32_t mode, const int32_t* draft_ids,
                        int32_t* accepted_len, int32_t* emitted, void* workspace,
                        size_t workspace_bytes, void* stream);

/* llima_verify_greedy over target rows held in split buffers (the layout of
 * llima_argmax_splits, B*(D+1) rows, sequence-major); the workspace is
 * llima_verify_greedy_workspace_bytes(B, D, sum of the widths, dtype). */
int llima_verify_greedy_splits(const void* const* splits, const int32_t* split_widths,
                               const int64_t* split_row_strides, int32_t n_splits, int32_t dtype,
                               int32_t B, int32_t D, int32_t mode, const int32_t* draft_ids,
                               int32_t* accepted_len, int32_t* emitted, void* workspace,
                               size_t workspace_bytes, void* stream);

/* Tree verification: K tree rows of logits [K][V]; retrieve_indices and
 * candidates [n_paths][L] int32 (device).  out[3] = {best path, accept length,
 * bonus token}. */
size_t llima_verify_tree_workspace_bytes(int32_t K, int32_t V, int32_t dtype);
int llima_verify_tree(const void* tree_logits, int32_t dtype, int32_t K, int32_t V,
                      const int32_t* retrieve_indices, const int32_t* candidates,
                      int32_t n_paths, int32_t L, int32_t* out, void* workspace,
                      size_t workspace_bytes, void* stream);

/* Stochastic speculative verification (rejection sampling) of B sequences with
 * D drafts: target_logits [B][D+1][V] fp32, draft_logits [B][D][V] fp32,
 * draft_ids [B][D], u_accept [B][D], u_resample [B].  Accept draft k iff
 * p_t(x_k) >= u_k * p_d(x_k); at the first rejection resample from
 * max(0, p_t - p_d); after D acceptances draw a bonus token from p_t[D].
 * Probabilities are fixed-point softmax weights built per chunk of 8192 ids
 * (W_i = rint(exp(x_i - m_c) 2^36) * rint(exp(m_c - M) 2^27), m_c the chunk's
 * maximum, M the row's), so each row is read once with no wait between
 * workgroups; the draws use W_i >> 32.  V % 4 == 0, V <= 2^22, D <= 255, rows
 * 16-byte aligned. */
size_t llima_verify_rejection_workspace_bytes(int32_t B, int32_t D, int32_t V);
int llima_verify_rejection(const float* target_logits, const float* draft_logits, int32_t B,
                           int32_t D, int32_t V, const int32_t* draft_ids,
                           const float* u_accept, const float* u_resample,
                           int32_t* accepted_len, int32_t* emitted, void* workspace,
                           size_t workspace_bytes, void* stream);


/* Log-likelihood of B target tokens: replaces score_logits
 * (sima_lmm/devkit/cpp/language_model.cpp:29-62), one row per call there.
 * targets [B] int32 (device).  out_logprob[B] (double) = x_t - (max + log sum
 * exp(x - max)); NaN when the row holds a NaN or its maximum is infinite (as
 * the reference's double sum).  out_is_greedy[B] = 1 when the target is the
 * first maximum, else 0; a target outside [0, V) (the reference throws
 * std::runtime_error) gives LLIMA_E_RANGE there and a NaN log-probability. */
size_t llima_score_logits_workspace_bytes(int32_t B, int32_t V, int32_t dtype);
int llima_score_logits(const void* logits, int32_t dtype, int32_t B, int32_t V,
                       int64_t row_stride, const int32_t* targets, double* out_logprob,
                       int32_t* out_is_greedy, void* workspace, size_t workspace_bytes,
                       void* stream);

/* Gemma4 MTP masked argmax of B rows: replaces select_candidate_tokens
 * (sima_lmm/devkit/cpp/gemma4_mtp_helpers.cpp:113-167) and
 * LanguageModel::_argmax_gemma4_mtp_masked_row
 * (sima_lmm/devkit/cpp/language_model_gemma4_mtp.cpp:31-97).
 * centroid_logits: bf16 [B][centroid_stride] (C used, C <= 8192);
 * token_ordering: [V] token ids, V / C per centroid; the top_k centroids by
 * (value desc, index asc) give the candidate tokens, and out_ids[B] receives
 * the candidate with the greatest logit (lowest token id on equal values; NaN
 * never selected).  logits may be NULL (selection only).  out_candidates
 * (nullable, [B][top_k * V / C]) receives the candidates in the reference's
 * order (centroid rank, then ordering position).  out_status (nullable, [B]):
 * LLIMA_OK, LLIMA_E_RANGE for an ordering entry >= V among the candidates, or
 * LLIMA_E_INVAL when no candidate has a non-NaN logit (both are
 * std::runtime_error in the reference); out_ids is then -1.  Returns
 * LLIMA_E_INVAL when V is not a multiple of C or top_k is outside [1, C]
 * (the reference's own checks). */
size_t llima_mtp_masked_argmax_workspace_bytes(int32_t B);
int llima_mtp_masked_argmax(const uint16_t* centroid_logits, int64_t centroid_stride, int32_t C,
                            const uint32_t* token_ordering, int32_t top_k, const void* logits,
                            int32_t dtype, int32_t B, int32_t V, int64_t row_stride,
                            int32_t* out_ids, int32_t* out_status, uint32_t* out_candidates,
                            void* workspace, size_t workspace_bytes, void* stream);

/* LM head with a fused softcap and argmax, for decode-sized batches: for each
 * of B hidden rows (bf16 [B][H], 16-byte aligned) and V vocab rows of the
 * weight (bf16 [V][H], the nn.Linear layout, 16-byte aligned),
 *   logit = round(softcap * tanh(s / softcap))  (s when softcap <= 0),
 *   s = sum_h hidden[b][h] * weight[v][h]  in fp32,
 * where round is to the nearest bf16 (ties to even) for logit_dtype
 * LLIMA_BF16 -- the precision of the reference's executed graphs
 * (sima_lmm/model/model_graph.py:30-45), so logits equal in bf16 tie and the
 * lower index wins -- and none for LLIMA_F32.  out_ids[B] = first index of the
 * maximum logit (NaN never wins; a row with no non-NaN logit gives 0),
 * out_vals[B] (nullable) its value, out_logits (nullable, fp32 [B][V], or bf16
 * with LLIMA_LOGITS_OUT_BF16) every logit.  H % 8 == 0, and H <= 4096 unless H % 64 == 0 (then H <= 65536).  The
 * weights are read once per 8 hidden rows (H <= 2048) or 4 (H <= 4096); wider
 * batches, and rows wider than 4096, use MFMA tiles that read them once per 256
 * rows (H % 64 == 0). */
size_t llima_lm_head_argmax_workspace_bytes(int32_t B, int32_t V);
int llima_lm_head_argmax(const void* hidden, const void* weight, int32_t B, int32_t H, int32_t V,
                         float softcap, int32_t logit_dtype, int32_t* out_ids, float* out_vals,
                         float* out_logits, void* workspace, size_t workspace_bytes, void* stream);

/* The same LM head over a weight prepacked once (at model load) by
 * llima_lm_head_pack: llima_lm_head_packed_bytes(V, H) bytes (0: H is not a
 * multiple of 256 or exceeds 65536), 16-byte aligned, holding the bf16 [V, H]
 * weight in the MFMA's operand order (32 vocab rows x 16 ids per 1 KB, zero
 * rows up to a multiple of 32; for each 128 ids, the row blocks in order).  llima_lm_head_argmax_packed takes the packed
 * weight in place of `weight` and gives the same ids, values and logits as
 * llima_lm_head_argmax's MFMA tiles; it reads the weight once per 64 hidden
 * rows, each wave streaming contiguous memory.  Workspace:
 * llima_lm_head_argmax_packed_workspace_bytes(B, H, V) (0 for invalid sizes).  No counterpart in the reference,
 * whose LM head runs inside its compiled graph (language_part_base.py:171-180):
 * a weight layout chosen at load time, as such graphs choose theirs. */
size_t llima_lm_head_packed_bytes(int32_t V, int32_t H);
size_t llima_lm_head_argmax_packed_workspace_bytes(int32_t B, int32_t H, int32_t V);
int llima_lm_head_pack(const void* weight, int32_t V, int32_t H, void* packed, size_t packed_bytes,
                       void* stream);
int llima_lm_head_argmax_packed(const void* hidden, const void* packed, int32_t B, int32_t H,
                                int32_t V, float softcap, int32_t logit_dtype, int32_t* out_ids,
                                float* out_vals, float* out_logits, void* workspace,
                                size_t workspace_bytes, void* stream);

/* LM head with a fused scoring epilogue: the log-likelihood of B target
 * tokens under the LM head's logits, as llima_lm_head_argmax computes them
 * (same softcap, logit_dtype LLIMA_BF16 or LLIMA_F32 rounding, same kernels),
 * without writing or reading the [B][V] logits: the head's epilogue keeps,
 * per wave and hidden row, its maximum and sum of exp(logit - maximum) beside
 * the argmax key, and a per-row finish combines them in double.  Replaces the
 * LM head followed by score_logits (sima_lmm/devkit/cpp/language_model.cpp:29-62;
 * the reference scores the logits its graph wrote,
 * sima_lmm/model/language_part_base.py:157-180).  targets [B] int32 (device);
 * out_logprob [B] and out_is_greedy [B] as llima_score_logits (NaN with a NaN
 * logit or an infinite maximum; LLIMA_E_RANGE and NaN for a target outside
 * [0, V)).  The log-probability agrees with llima_score_logits over the same
 * logits to about 1e-6 (fp32 exp terms, double combination); the flag is
 * exact.  LLIMA_LOGITS_OUT_BF16 is rejected (no logits output).  Sizes,
 * alignment and the _packed form (a weight from llima_lm_head_pack) as the
 * argmax entry points. */
size_t llima_lm_head_score_workspace_bytes(int32_t B, int32_t V);
int llima_lm_head_score(const void* hidden, const void* weight, int32_t B, int32_t H, int32_t V,
                        float softcap, int32_t logit_dtype, const int32_t* targets,
                        double* out_logprob, int32_t* out_is_greedy, void* workspace,
                        size_t workspace_bytes, void* stream);
size_t llima_lm_head_score_packed_workspace_bytes(int32_t B, int32_t H, int32_t V);
int llima_lm_head_score_packed(const void* hidden, const void* packed, int32_t B, int32_t H,
                               int32_t V, float softcap, int32_t logit_dtype,
                               const int32_t* targets, double* out_logprob,
                               int32_t* out_is_greedy, void* workspace, size_t workspace_bytes,
                               void* stream);

/* LM head with greedy chain verification fused: for B sequences of D + 1
 * hidden rows each (hidden bf16 [B][D+1][H]), the head's argmax of every row
 * (as llima_lm_head_argmax: softcap, logit_dtype rounding, NaN never wins),
 * then the chain rule of llima_verify_greedy on those ids: accepted_len[B] =
 * the length of the prefix where draft_ids[b][k] equals row k's argmax;
 * emitted[B][D+1] = the accepted drafts, then row accepted_len's argmax (the
 * correction or the bonus token), then -1.  Replaces the verification step's
 * LM head, its logits and _argmax_lm_head_rows + resolve_draft_tokens
 * (sima_lmm/devkit/cpp/language_model.cpp:3636-3687,
 * sima_lmm/devkit/cpp/gemma4_mtp_helpers.cpp:81-111): no [B(D+1)][V] logits are
 * written.  Sizes and alignment as llima_lm_head_argmax (its B is B (D + 1));
 * the _packed form takes a weight from llima_lm_head_pack.
 * LLIMA_LOGITS_OUT_BF16 is rejected. */
size_t llima_lm_head_verify_greedy_workspace_bytes(int32_t B, int32_t D, int32_t V);
int llima_lm_head_verify_greedy(const void* hidden, const void* weight, int32_t B, int32_t D,
                                int32_t H, int32_t V, float softcap, int32_t logit_dtype,
                                const int32_t* draft_ids, int32_t* accepted_len,
                                int32_t* emitted, void* workspace, size_t workspace_bytes,
                                void* stream);
size_t llima_lm_head_verify_greedy_packed_workspace_bytes(int32_t B, int32_t D, int32_t H,
                                                         int32_t V);
int llima_lm_head_verify_greedy_packed(const void* hidden, const void* packed, int32_t B,
                                       int32_t D, int32_t H, int32_t V, float softcap,
                                       int32_t logit_dtype, const int32_t* draft_ids,
                                       int32_t* accepted_len, int32_t* emitted, void* workspace,
                                       size_t workspace_bytes, void* stream);

/* LM head with EAGLE3 tree verification fused: the head's argmax of each of
 * the K tree rows (hidden bf16 [K][H]; a row whose greatest logit does not
 * exceed -inf gives 0, as the reference's scan from -inf), then
 * llima_verify_tree's gather and evaluate_posterior: out[3] = {best path,
 * accept length, bonus token}.  Replaces the tree step's LM head, its logits
 * and the verify argmax + tree_decoding + evaluate_posterior
 * (sima_lmm/devkit/cpp/language_model_eagle3.cpp:486-567,
 * sima_lmm/devkit/cpp/eagle_helpers.hpp:153-195): no [K][V] logits are
 * written.  Sizes and alignment as llima_lm_head_argmax; the _packed form
 * takes a weight from llima_lm_head_pack.  LLIMA_LOGITS_OUT_BF16 is rejected. */
size_t llima_lm_head_verify_tree_workspace_bytes(int32_t K, int32_t V);
int llima_lm_head_verify_tree(const void* hidden, const void* weight, int32_t K, int32_t H,
                              int32_t V, float softcap, int32_t logit_dtype,
                              const int32_t* retrieve_indices, const int32_t* candidates,
                              int32_t n_paths, int32_t L, int32_t* out, void* workspace,
                              size_t workspace_bytes, void* stream);
size_t llima_lm_head_verify_tree_packed_workspace_bytes(int32_t K, int32_t H, int32_t V);
int llima_lm_head_verify_tree_packed(const void* hidden, const void* packed, int32_t K,
                                     int32_t H, int32_t V, float softcap, int32_t logit_dtype,
                                     const int32_t* retrieve_indices, const int32_t* candidates,
                                     int32_t n_paths, int32_t L, int32_t* out, void* workspace,
                                     size_t workspace_bytes, void* stream);

/* Heap top-k of each of `rows` rows of `cols` values (row r at x + r*row_stride
 * elements), exactly as topk<T> (sima_lmm/devkit/cpp/utils.hpp:216-281):
 * a min-heap of the first k values, replaced at the root only by strictly
 * greater values, output by a selection sort of the heap -- the same indices in
 * the same order, ties included.  k in [1, 32], cols >= k.  out_idx [rows][k]
 * int32, out_vals [rows][k] fp32 (bf16 values widened exactly).  No workspace. */
int llima_topk(const void* x, int32_t dtype, int32_t rows, int32_t cols, int64_t row_stride,
               int32_t k, int32_t* out_idx, float* out_vals, void* stream);

/* EAGLE3 draft tree (the selection side of topk_generate,
 * sima_lmm/devkit/cpp/language_model_eagle3.cpp:808-1164).  The caller runs the
 * draft model between the calls; `tree` is a caller-owned device buffer of
 * llima_eagle3_tree_bytes(K, depth) bytes holding the tree from begin to finish
 * (K = the draft's top-k, 1..32; depth = levels, 1..16; the reference uses K = 5,
 * depth 4).  d2t: int32 [Vd] draft-to-target offsets (token = id + d2t[id]).
 *   begin:  the root row [Vd]: its top K ids (topk), their log-softmax (the
 *           level's scores), out_input_ids [K] = their tokens.
 *   grow:   level = 1 .. depth-1, logits [K][Vd] (row stride row_stride): each
 *           row's top K and log-softmax plus that row's score, the best K of the
 *           K*K cumulative scores (topk); out_input_ids [K] their tokens,
 *           out_parent_rows [K] (nullable) their rows, out_mask (nullable,
 *           fp32 [K][K*(level+1)]) the draft attention mask for the next level.
 *   finish: after the depth-1 grow calls: the best total_tokens (1..32) node
 *           scores; out_tokens [N] (N = total_tokens + 1: sample_token, then the
 *           survivors' tokens in node order), out_tree_mask fp32 [N][N],
 *           out_position_ids [N], out_retrieve [N][N] (leaf paths from the
 *           root, -1 padded), out_dims [2] = {leaf paths, columns used}.
 * log-softmax uses exp and log rounded once from double (the correctly rounded
 * values; the reference's C library expf/logf agree on all but rare arguments). */
size_t llima_eagle3_tree_bytes(int32_t K, int32_t depth);
int llima_eagle3_tree_begin(const void* logits, int32_t dtype, int32_t Vd, const int32_t* d2t,
                            int32_t K, int32_t depth, void* tree, size_t tree_bytes,
                            int32_t* out_input_ids, void* stream);
int llima_eagle3_tree_grow(const void* logits, int32_t dtype, int32_t Vd, int64_t row_stride,
                           const int32_t* d2t, int32_t K, int32_t depth, int32_t level,
                           void* tree, size_t tree_bytes, int32_t* out_input_ids,
                           int32_t* out_parent_rows, float* out_mask, void* stream);
int llima_eagle3_tree_finish(void* tree, size_t tree_bytes, int32_t K, int32_t depth,
                             int32_t total_tokens, int32_t sample_token, int32_t* out_tokens,
                             float* out_tree_mask, int32_t* out_position_ids,
                             int32_t* out_retrieve, int32_t* out_dims, void* stream);

/* Stop-token check of B sequences' newly emitted tokens [B][M] (count[B]
 * valid per sequence, nullable: all M), as the reference's decode loops do it:
 * the run is cut at room[b] tokens (the cache space left; nullable: no cap) and
 * after its first token in the stop set, which is kept.  stop_mask: the stop
 * set as a bitmask over V ids ([ceil(V/32)] uint32, bit id & 31 of word id >> 5,
 * LSB first); ids outside [0, V) never stop.  out_keep[B]: tokens to keep;
 * out_status[B] (nullable): LLIMA_STOP_TOKEN when a stop token ended the run,
 * else LLIMA_STOP_CACHE_FULL when the run reached room[b] (cut there, or
 * filling it exactly: language_model_gemma4_mtp.cpp:953-955, 1011-1012), else
 * LLIMA_STOP_NONE. */
enum { LLIMA_STOP_NONE = 0, LLIMA_STOP_TOKEN = 1, LLIMA_STOP_CACHE_FULL = 2 };
int llima_stop_check(const int32_t* tokens, const int32_t* count, int32_t B, int32_t M,
                     const uint32_t* stop_mask, int32_t V, const int32_t* room,
                     int32_t* out_keep, int32_t* out_status, void* stream);

const char* llima_status_string(int status);
int llima_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* LLIMA_SAMPLER_H */
