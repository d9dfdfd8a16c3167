"""llima_amd -- MI355X-native logits -> token selection (sampling and draft
verification) for an LLiMa-style decode loop.  Compute is in hand-written HIP
kernels (libllima_sampler.so, C ABI in include/llima_sampler.h)."""
from .sampler import (Eagle3DraftTree, SamplerConfig, Workspace, topk, argmax, argmax_bf16,
                      argmax_gemma4_mtp_masked_row, argmax_gemma4_mtp_masked_rows,
                      argmax_lm_head_rows, calc_next_token_id, lm_head_argmax, lm_head_pack, lm_head_score, lm_head_verify_greedy, lm_head_verify_tree,
                      PackedLmHead, resolve_draft_tokens, sample,
                      score_logits, select_candidate_tokens, spec_path_argmax, stop_check,
                      stop_mask, verify_greedy,
                      verify_rejection, verify_tree)

__all__ = ["Eagle3DraftTree", "topk", "SamplerConfig", "Workspace", "argmax", "argmax_bf16", "argmax_gemma4_mtp_masked_row",
           "argmax_gemma4_mtp_masked_rows", "argmax_lm_head_rows", "calc_next_token_id", "lm_head_argmax", "lm_head_score", "lm_head_verify_greedy", "lm_head_verify_tree",
           "lm_head_pack", "PackedLmHead",
           "resolve_draft_tokens", "sample", "score_logits", "select_candidate_tokens", "spec_path_argmax", "stop_check", "stop_mask",
           "verify_greedy", "verify_rejection", "verify_tree"]
