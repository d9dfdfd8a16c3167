"""Writes reference_vectors.json: the known-answer vectors of the reference's own
runtime unit test tests/runtime/gemma4_mtp_helpers_test.cpp (sima-neat/llima),
transcribed as data (inputs and expected outputs only):
  select_candidate_tokens  :89-135
  resolve_draft_tokens     :183-245
Run: python tests/golden/make_reference_vectors.py
"""
import json
import os

VECTORS = {
    "select_candidate_tokens": [
        # test_selects_tokens_from_the_highest_scoring_centroids (:89-101)
        {"centroid_logits": [1.0, 10.0, 2.0, 9.0], "token_ordering": [0, 1, 4, 5, 2, 3, 6, 7],
         "top_k": 2, "expected": [4, 5, 6, 7]},
        # test_centroid_ties_use_the_lower_index_first (:103-115)
        {"centroid_logits": [1.0, 10.0, 2.0, 10.0], "token_ordering": [0, 1, 7, 5, 2, 3, 6, 4],
         "top_k": 2, "expected": [7, 5, 6, 4]},
    ],
    "select_candidate_tokens_errors": [
        # test_rejects_invalid_metadata (:117-135)
        {"centroid_logits": [0.0, 0.0, 0.0, 0.0], "token_ordering": [0, 1, 2, 3, 4, 5, 6, 7],
         "top_k": 0},
        {"centroid_logits": [0.0, 0.0, 0.0, 0.0], "token_ordering": [8, 1, 2, 3, 4, 5, 6, 7],
         "top_k": 4},
    ],
    "resolve_draft_tokens": [
        # test_verification_emits_the_first_target_mismatch (:183-197)
        {"drafts": [10, 11, 12, 13, 14, 15], "targets": [10, 21, 22, 23, 24, 25, 26],
         "expected": [[10, True], [21, False]]},
        # test_verification_emits_target_token_without_drafts (:199-208)
        {"drafts": [], "targets": [21], "expected": [[21, False]]},
        # test_verification_accepts_an_early_exit_result (:210-218)
        {"drafts": [10, 11, 12, 13, 14, 15], "targets": [10, 21],
         "expected": [[10, True], [21, False]]},
        # test_verification_emits_bonus_after_a_full_match (:220-236)
        {"drafts": [10, 11, 12, 13, 14, 15], "targets": [10, 11, 12, 13, 14, 15, 16],
         "expected": [[10, True], [11, True], [12, True], [13, True], [14, True], [15, True],
                      [16, False]]},
    ],
    "resolve_draft_tokens_errors": [
        # test_verification_rejects_an_incomplete_target_result (:238-245)
        {"drafts": [10, 11], "targets": [10, 11]},
    ],
}

if __name__ == "__main__":
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_vectors.json")
    with open(out, "w") as f:
        json.dump(VECTORS, f, indent=1)
    print(out)
