"""Llama-3 family front-end: scales stored in the input dtype."""
