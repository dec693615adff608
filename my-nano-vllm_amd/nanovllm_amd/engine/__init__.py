"""Host-side metadata and decode-graph runner."""
