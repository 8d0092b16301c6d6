"""GPU layer of the MI355X backend; `from simple_llm_amd.gpu import gpu` mirrors
the reference's `from gpu import gpu` (simple-llm/src/gpu_test.py:16)."""
