"""Host-framework models whose attention the ChronoQuant patch re-routes."""
