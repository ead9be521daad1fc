"""Writes tests/golden/reference_vectors.json: the known-answer vectors and literal expected values that
the reference's own tests hold for this path, restated as data (nothing from the reference is imported or
run).  Sources:
  * Philox4x32-10 known-answer vectors of Random123 (the reference checks its philox against them:
    engine/include/mtp.h:134 smk_test_philox; the three published Random123 known answers);
  * vLLM / sglang / llama.cpp penalty cases: tests/test_logit_procs.py:178-221;
  * llama.cpp min_p cases: tests/test_logit_procs.py:266-273;
  * chi-square survival values: tests/test_spec_procs.py:153.
"""
import json
from pathlib import Path

V = {
    "philox_kat": [
        {"ctr": [0, 0, 0, 0], "key": [0, 0], "out": [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]},
        {"ctr": [0xFFFFFFFF] * 4, "key": [0xFFFFFFFF] * 2, "out": [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]},
        {"ctr": [0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], "key": [0xA4093822, 0x299F31D0],
         "out": [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]},
    ],
    # tests/test_logit_procs.py:196-205 (sglang test_penaltylib.py): processed logit values
    "sglang": [
        {"logits": 0.0, "gen": [5], "frequency": 2.0, "check": {"5": -2.0, "0": 0.0}},
        {"logits": 0.0, "gen": [3, 3], "frequency": 1.0, "check": {"3": -2.0}},
        {"logits": 0.0, "gen": [7, 7], "presence": 1.0, "check": {"7": -1.0}},
    ],
    # tests/test_logit_procs.py:216-221 (llama.cpp test_penalties): softmax of 5 tokens at log(0.2), -inf elsewhere
    "llama_penalties": [
        {"gen": [0], "repetition": 50.0, "probs": [0, 0.25, 0.25, 0.25, 0.25], "tol": 2e-6},
        {"gen": [0, 1, 2], "repetition": 50.0, "probs": [0, 0, 0, 0.5, 0.5], "tol": 2e-6},
        {"gen": [0, 1, 2, 0, 0], "repetition": 50.0, "probs": [0, 0, 0, 0.5, 0.5], "tol": 2e-6},
        {"gen": [0], "frequency": 5.0, "presence": 5.0, "probs": [0.000011, 0.249997, 0.249997, 0.249997, 0.249997], "tol": 2e-6},
        {"gen": [0, 1, 2], "frequency": 5.0, "presence": 5.0, "probs": [0.000023, 0.000023, 0.000023, 0.499966, 0.499966], "tol": 2e-6},
        {"gen": [0, 1, 2, 0, 0], "frequency": 5.0, "presence": 5.0, "probs": [0.0, 0.000023, 0.000023, 0.499977, 0.499977], "tol": 2e-6},
    ],
    # tests/test_logit_procs.py:266-273 (llama.cpp test_min_p): probabilities {.1,.2,.3,.4}, survivors renormalised
    "llama_min_p": [
        {"min_p": 0.0, "probs": [0.1, 0.2, 0.3, 0.4]},
        {"min_p": 0.24, "probs": [0.1, 0.2, 0.3, 0.4]},
        {"min_p": 0.26, "probs": [0.2 / 0.9, 0.3 / 0.9, 0.4 / 0.9]},
        {"min_p": 0.49, "probs": [0.2 / 0.9, 0.3 / 0.9, 0.4 / 0.9]},
        {"min_p": 0.51, "probs": [0.3 / 0.7, 0.4 / 0.7]},
        {"min_p": 0.74, "probs": [0.3 / 0.7, 0.4 / 0.7]},
        {"min_p": 0.76, "probs": [1.0]},
        {"min_p": 1.0, "probs": [1.0]},
    ],
    # tests/test_spec_procs.py:153: chi-square survival function known values
    "chi2_sf": [{"x": 10.0, "dof": 5, "sf": 0.0752352, "tol": 1e-6}, {"x": 3.84146, "dof": 1, "sf": 0.05, "tol": 1e-5},
                {"x": 101.879, "dof": 80, "sf": 0.05, "tol": 1e-4}],
}

if __name__ == "__main__":
    out = Path(__file__).resolve().parent / "reference_vectors.json"
    out.write_text(json.dumps(V, indent=1))
    print(out)
