"""Host-side mirror of the reference's ``model`` package interfaces for the
forecast-guided sparse attention path, backed by libsparda's HIP kernels."""
