"""MI355X-native sparse expert reader (drop-in for calibration_free_moe.reader)."""
