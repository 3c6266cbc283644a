"""miniMoE inference engine: MI355X-native paged-KV decode path."""
