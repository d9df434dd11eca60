"""End-to-end measurement harness: a random-init decoder model and a minimal
token-budgeted generation loop that drive the paged-attention operator the
way the reference's Engine / ModelRunner do (engine.py:33-56,
model_runner.py:236-287). It exists to measure and check the operator's
callers (output tokens per second, greedy-token parity), not as a serving
engine."""

from micro_vllm_amd.harness.engine import GenerationEngine, GenerationResult, Request  # noqa: F401
from micro_vllm_amd.harness.model import DecoderConfig, DecoderModel  # noqa: F401
