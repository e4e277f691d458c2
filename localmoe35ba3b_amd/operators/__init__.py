"""Operator layer: drop-in replacements for qwen35_deploy.operators."""
