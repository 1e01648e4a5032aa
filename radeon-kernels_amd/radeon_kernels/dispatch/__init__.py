"""Built-in dispatch manifests (JSON resources)."""
