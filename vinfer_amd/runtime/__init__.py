"""Callers of the sampler: the continuous-batching decode loop and its text stream."""

from vinfer_amd.runtime.batch import BatchDecoder, DecodeModel, SpeculativeDecoder, Step, check_request
from vinfer_amd.runtime.text import TextStream

__all__ = ["BatchDecoder", "DecodeModel", "SpeculativeDecoder", "Step", "TextStream", "check_request"]
