from .hf import ensure_local_model_path, load_config_dict, load_hf_weights_into_model

__all__ = ["ensure_local_model_path", "load_config_dict", "load_hf_weights_into_model"]
