"""Mirror of the reference package layout (vllm_gr/v1/attention)."""
