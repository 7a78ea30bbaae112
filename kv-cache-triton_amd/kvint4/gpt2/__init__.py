"""GPT-2 family front-end: scales and dequantized values always fp16."""
