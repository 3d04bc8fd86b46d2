"""libcmol_amd: MI355X-native decode hot path of libcmol behind its C API."""
