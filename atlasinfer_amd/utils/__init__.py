"""Host-side utilities around the quantized path (weight streaming)."""
