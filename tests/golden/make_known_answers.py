"""Writes reference_known_answers.json: input/expected values transcribed
from gorch's own test files for the hot path (data, with the file:line each
came from). Run from the repo root: python tests/golden/make_known_answers.py
"""
import json
import os

KA = {
    "bf16_roundtrip_exact": {
        "source": "bf16_test.go:13-25 (values with the low 16 bits stripped round-trip exactly)",
        "inputs": [0.0, 1.0, -1.0, 0.5, -0.5, 256.0, 1e-10, -1e10],
    },
    "bf16_roundtrip_approx": {
        "source": "bf16_test.go:30-39 (relative error <= 1/128)",
        "inputs": [0.123456, -0.987654, 3.14159, 2.71828, 0.001234],
        "max_rel": 1.0 / 128.0,
    },
    "bf16_special": {
        "source": "bf16_test.go:42-57 (0, +Inf, -Inf survive)",
        "inputs": ["0", "inf", "-inf"],
    },
    "bf16_integers": {
        "source": "bf16_test.go:86-104 (whole integers <= 256 are exact)",
        "inputs": [1, 2, 3, 4, 5, 6],
    },
    "bf16_safetensors_values": {
        "source": "model/safetensors_bf16_test.go:21-24 (0.1 and 1e-3 not representable, 1.5 and -2 are)",
        "inputs": [0.1, 1.5, -2.0, 1e-3, 3.14159, -0.4567],
        "representable": [False, True, True, False, False, False],
    },
    "rmsnorm_spec": {
        "source": "nn/rmsnorm_test.go:12-34 (eps = 0, gamma = 1, tolerance 1e-5)",
        "x": [[1, 2, 3, 4], [-1, 0, 1, 2]],
        "want": [[1 / 2.7386128, 2 / 2.7386128, 3 / 2.7386128, 4 / 2.7386128],
                 [-1 / 1.2247449, 0 / 1.2247449, 1 / 1.2247449, 2 / 1.2247449]],
        "tol": 1e-5,
    },
    "bf16_matmul_probe": {
        "source": "bf16_matmul.go:63-112 (16x16x16 probe: a[i] = (i%7)*0.25-0.75, "
                  "b[i] = ((i*5)%11)*0.125-0.625, row-major; |GPU - CPU| <= 1e-3)",
        "n": 16,
        "tol_abs": 1e-3,
    },
}

if __name__ == "__main__":
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_known_answers.json")
    with open(out, "w") as f:
        json.dump(KA, f, indent=1)
    print(out)
