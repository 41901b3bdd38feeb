from .group_config import QuantConfig, GROUPS  # noqa: F401
