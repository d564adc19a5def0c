"""Producer side of the AutoAWQ format: group-wise int4 quantization and packing on the GPU."""
