class _Registry:
    def get_implementation(self, name, backend="eager"):
        if backend != "eager":
            raise KeyError(backend)
        from .backends import eager
        return getattr(eager, name)


registry = _Registry()
