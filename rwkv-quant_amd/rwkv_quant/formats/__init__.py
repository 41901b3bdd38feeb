"""`.rwkvq` format: container, bit layouts, writer, reader."""
