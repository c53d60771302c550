"""Model integration (reference: integration/)."""
