"""TokenVector MI355X-native packages."""
