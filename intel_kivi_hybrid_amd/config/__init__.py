from .model_config import detect_model_config

__all__ = ["detect_model_config"]
