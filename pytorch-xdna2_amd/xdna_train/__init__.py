"""MI355X-native ``xdna`` PrivateUse1 backend (placeholder until the device module lands)."""
__version__ = "0.1.0"
