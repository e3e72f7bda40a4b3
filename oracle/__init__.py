"""CPU oracle for the fused KAN hot path (test infrastructure, never the product).

``kan64`` is the float64 NumPy restatement of the reference's algorithm;
``torch_cpu`` is the plain-ops torch-CPU route timed as the CPU baseline.
"""
