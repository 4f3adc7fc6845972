"""CPU oracle (test infrastructure only): float64 restatement of causal GQA attention. See attention.py."""
