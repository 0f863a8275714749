from .exporter import export_pytorch  # noqa: F401
