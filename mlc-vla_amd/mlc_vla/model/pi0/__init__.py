from .pi0_config import GemmaExpertConfig, Pi0Config, SiglipConfig  # noqa: F401
