"""Engine-side producers of the attention metadata."""

from voiceagent_amd.engine.metadata import (DecodeGraphMetadata, SequenceState, prepare_batch,
                                            slot_of)

__all__ = ["DecodeGraphMetadata", "SequenceState", "prepare_batch", "slot_of"]
