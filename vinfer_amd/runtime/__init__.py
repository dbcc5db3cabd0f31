"""Callers of the sampler: the continuous-batching decode loop."""

from vinfer_amd.runtime.batch import BatchDecoder, DecodeModel, SpeculativeDecoder, Step, TextStream, check_request

__all__ = ["BatchDecoder", "DecodeModel", "SpeculativeDecoder", "Step", "TextStream", "check_request"]
