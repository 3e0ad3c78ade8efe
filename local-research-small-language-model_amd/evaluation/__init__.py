"""Routing-quality evaluation (evaluation/forecast_metrics.py of the reference)."""
