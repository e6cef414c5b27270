"""Minimal stand-in for the parts of vLLM that knlp_amd.vllm_backend imports.

vLLM is not installed in this environment; these tests only exercise the
backend's own logic (cache planning, write and decode dispatch, the
MIN_FUSED_SEQ_LEN gate, mixed-batch placement).  Test infrastructure only."""
