"""Serving-side batch execution (reference cortex/serve): the inference worker."""

from cortex.serve.worker import InferenceWorker, batch_bucket, event_bucket, load_model

__all__ = ["InferenceWorker", "batch_bucket", "event_bucket", "load_model"]
