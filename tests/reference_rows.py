"""The reference's executor row and key types, restated field for field for the executor-seam tests
(executor/rows.py:16-224, contract/stage.py:39-65, contract/rng.py:15-17): the adapters are driven
with values of exactly these shapes, as Executor._replay_stage (executor/executor.py:252-285) hands
them over.  Field names and meaning only; the reference's own validation is not restated."""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum

import torch


class CodePredictorSamplerRoute(str, Enum):
    FUSED = "fused"
    GENERAL = "general"


@dataclass(frozen=True, slots=True)
class TalkerPrefillCaptureKey:
    capture_batch_size: int
    token_capacity: int
    capture_sequence_length: int | None


@dataclass(frozen=True, slots=True)
class TalkerDecodeCaptureKey:
    capture_batch_size: int


@dataclass(frozen=True, slots=True)
class CodePredictorCaptureKey:
    capture_batch_size: int


@dataclass(frozen=True, slots=True)
class TalkerSamplingExecutionRow:
    temperature: float
    top_k: int
    top_p: float
    repetition_penalty: float
    seed: int
    offset: int
    seen_token_mask: torch.Tensor | None


@dataclass(frozen=True, slots=True)
class TalkerPrefillExecutionRow:
    text_token_ids: torch.Tensor
    codec_token_ids: torch.Tensor
    codec_token_mask: torch.Tensor
    suppress_eos: bool
    sampling: TalkerSamplingExecutionRow


@dataclass(frozen=True, slots=True)
class TalkerDecodeExecutionRow:
    talker_step_embed: torch.Tensor
    text_token_id: torch.Tensor
    suppress_eos: bool
    sampling: TalkerSamplingExecutionRow


@dataclass(frozen=True, slots=True)
class TalkerPrefillRowsExecutionInput:
    request_ids: tuple[str, ...]
    rows: tuple[TalkerPrefillExecutionRow, ...]


@dataclass(frozen=True, slots=True)
class TalkerDecodeRowsExecutionInput:
    request_ids: tuple[str, ...]
    rows: tuple[TalkerDecodeExecutionRow, ...]
    reuse_attention_plan: bool = False


@dataclass(frozen=True, slots=True)
class CodePredictorExecutionRow:
    layer0_token: torch.Tensor
    past_hidden: torch.Tensor
    temperature: float
    top_k: int
    top_p: float
    seed: int
    offsets: tuple[int, ...]
    position_ids: torch.Tensor | None = None


@dataclass(frozen=True, slots=True)
class CodePredictorRowsExecutionInput:
    rows: tuple[CodePredictorExecutionRow, ...]
    sampler_route: CodePredictorSamplerRoute = CodePredictorSamplerRoute.FUSED


@dataclass(frozen=True, slots=True)
class CodePredictorInput:
    layer0_token: torch.Tensor
    past_hidden: torch.Tensor
    temperature: torch.Tensor
    top_k: torch.Tensor
    top_p: torch.Tensor
    seed: torch.Tensor
    offsets: torch.Tensor
    num_code_groups: int
    position_ids: torch.Tensor | None = None


def replay_stage(executor, expected_key: type, key, values):
    """Executor._replay_stage's contract (executor/executor.py:252-285): a key of the wrong type is
    refused before the executor sees it; otherwise the executor's replay runs."""

    if not isinstance(key, expected_key):
        raise TypeError("replay requires its typed capture key")
    return executor.replay(key, values)
