"""Python view of the MI355X batched token sampler (liboxide_sampler.so).

Four layers, all thin over the C ABI in include/oxide_sampler.h:

- `BatchSampler`: the batched device call, `oxs_sample_batch`, on torch
  tensors that already live on the GPU (the decode-loop form).
- `SamplingConfig`, `MirostatMode`, `SamplerState`, `AcademicSamplerEngine`:
  the reference's single-row API (crates/oxide-core/src/sampler.rs:15-390),
  same names and argument meaning, each call running one row on the GPU.
- `DfaSchemaGrammar`: the reference's grammar DFA (crates/oxide-core/src/dfa.rs),
  whose token masks run on the GPU (`oxs_dfa_mask`) and feed the sampler.
- `DecodeLoop`: the scheduler's decode stage
  (crates/oxide-engine/src/continuous_batching.rs:940-1040) with every
  sequence's sampler state on the device, one `oxs_decode_step` per step.

There is no CPU path: without the built library every call raises
`LibraryMissing`.
"""
from .engine import (
    AcademicSamplerEngine,
    BatchSampler,
    MirostatMode,
    SamplerState,
    SamplingConfig,
    ShapeMismatch,
    configs_to_array,
)
from .grammar import (DfaSchemaGrammar, GbnfGrammarEngine, GbnfRule, GrammarConstraintType, GrammarLogitMasker,
                      SchemaMismatch, StructuredOutputEngine, TokenBytes)
from .decode import DecodeLoop, TokenEvent
from .lm_head import LmHeadQ8_0, quantize_q8_1
from ._abi import (
    LibraryMissing,
    OxsError,
    load_library,
)

__all__ = [
    "AcademicSamplerEngine",
    "BatchSampler",
    "MirostatMode",
    "SamplerState",
    "SamplingConfig",
    "ShapeMismatch",
    "configs_to_array",
    "DfaSchemaGrammar",
    "GbnfGrammarEngine",
    "GbnfRule",
    "GrammarLogitMasker",
    "GrammarConstraintType",
    "StructuredOutputEngine",
    "SchemaMismatch",
    "TokenBytes",
    "DecodeLoop",
    "TokenEvent",
    "LmHeadQ8_0",
    "quantize_q8_1",
    "LibraryMissing",
    "OxsError",
    "load_library",
]
