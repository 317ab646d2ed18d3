"""MI355X-native paged-decode attention engine (hot path of a paged-KV serving engine)."""
