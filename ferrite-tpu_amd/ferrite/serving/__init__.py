from ferrite.serving.engine import Engine, ServeConfig, bucket_for, reference_greedy

__all__ = ["Engine", "ServeConfig", "bucket_for", "reference_greedy"]
