"""Serving-side batch execution (reference cortex/serve): the inference worker."""

from cortex.serve.worker import InferenceWorker, event_bucket, load_model

__all__ = ["InferenceWorker", "event_bucket", "load_model"]
