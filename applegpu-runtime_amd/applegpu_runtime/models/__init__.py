"""Model recipes on the applegpu_runtime op surface (reference: python/applegpu_runtime/models/)."""
