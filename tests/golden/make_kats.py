"""Writes elementwise_kats.json: the known-answer cases of the reference's
GPU elementwise test, as data.

Provenance (reference checkout, read as text):
  tests/test_gpu_elementwise.gd:31-35  broadcast shape cases (op, a, b)
  tests/test_gpu_elementwise.gd:36-38  unary shape cases
  tests/test_gpu_elementwise.gd:59     operands drawn from U(0.5, 3.5)
  tests/test_gpu_elementwise.gd:165-172 LeakyRelu alpha 0.2 known answers
  tests/test_gpu_elementwise.gd:175-181 Where with a scalar else-branch
  tests/test_gpu_elementwise.gd:199    absolute tolerance 1e-5
The reference's expected values for the shape cases come from an independent
coordinate walk (:64-95); tests/test_oracle.py re-implements that walk.
"""
import json
import os

KATS = {
    "source": "tests/test_gpu_elementwise.gd",
    "abs_tolerance": 1e-5,
    "operand_range": [0.5, 3.5],
    "binary_shape_cases": [
        ["Mul", [2, 3, 4], [3, 1]],
        ["Add", [5, 7], []],
        ["Sub", [4, 6], [4, 6]],
        ["Div", [2, 1, 5], [2, 4, 5]],
    ],
    "unary_shape_cases": [["Sqrt", [3, 9]], ["Sigmoid", [64]], ["Floor", [17]]],
    "leaky_relu": {"alpha": 0.2, "x": [-2.0, -0.5, 0.0, 0.5, 2.0],
                   "want": [-0.4, -0.1, 0.0, 0.5, 2.0]},
    "where": {"cond": [1.0, 0.0, 1.0, 0.0], "x": [10.0, 20.0, 30.0, 40.0], "y": [-1.0],
              "want": [10.0, -1.0, 30.0, -1.0]},
}

if __name__ == "__main__":
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "elementwise_kats.json")
    with open(path, "w") as f:
        json.dump(KATS, f, indent=1)
        f.write("\n")
    print("wrote", path)
