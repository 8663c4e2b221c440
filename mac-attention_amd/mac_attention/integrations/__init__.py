"""Framework integrations (SGLang)."""
