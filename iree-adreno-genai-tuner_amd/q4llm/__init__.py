"""MI355X (gfx950) int4 LLM hot path: C-ABI library bindings, the LlamaQ4 module API and the
llm_runner schedule. Kernels live in ../csrc and are built into ../lib/libq4llm.so."""

from ._lib import LIB, Q4Error  # noqa: F401
