"""A Python consumer of the bundles sparsewavecomp_amd.bundle produces: the
launch side of the lrrt runtime's Bundle::launch(n, args)
(README.md:111-140 in the reference), used by the GPU tests and by
bench.py to run a bundle the way lrrt would.

It follows the manifest exactly as a consumer would: evaluate the grid
expression (total work-items) for n, divide by the block, pack each
pointer at its recorded kernarg offset, and launch the named symbol from
its code object through the HIP module API of the HIP runtime torch already
loaded (so torch device pointers are valid)."""
import ctypes
import json
import struct
from pathlib import Path

from sparsewavecomp_amd.bundle import evaluate_grid

_hip = None


def hip():
    global _hip
    if _hip is None:
        import torch
        torch.cuda.init()
        path = None
        with open("/proc/self/maps") as f:
            for line in f:
                if "libamdhip64.so" in line:
                    path = line.split()[-1]
                    break
        if path is None:
            raise RuntimeError("libamdhip64 is not loaded")
        lib = ctypes.CDLL(path)
        lib.hipModuleLoadData.argtypes = [ctypes.POINTER(ctypes.c_void_p),
                                          ctypes.c_void_p]
        lib.hipModuleGetFunction.argtypes = [ctypes.POINTER(ctypes.c_void_p),
                                             ctypes.c_void_p, ctypes.c_char_p]
        lib.hipModuleLaunchKernel.argtypes = [
            ctypes.c_void_p] + [ctypes.c_uint] * 7 + [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        lib.hipModuleUnload.argtypes = [ctypes.c_void_p]
        _hip = lib
    return _hip


class Bundle:
    def __init__(self, directory):
        self.dir = Path(directory)
        self.manifest = json.loads((self.dir / "manifest.json").read_text())
        self.kernels = {k["name"]: k for k in self.manifest["kernels"]}
        self._modules = {}
        self._images = {}

    def _function(self, kernel):
        rel = kernel["code_object"]
        if rel not in self._modules:
            image = (self.dir / rel).read_bytes()
            buf = ctypes.create_string_buffer(image, len(image))
            self._images[rel] = buf
            mod = ctypes.c_void_p()
            rc = hip().hipModuleLoadData(ctypes.byref(mod), buf)
            if rc:
                raise RuntimeError(f"hipModuleLoadData failed: {rc}")
            self._modules[rel] = mod
        fn = ctypes.c_void_p()
        rc = hip().hipModuleGetFunction(ctypes.byref(fn), self._modules[rel],
                                        kernel["symbol"].encode())
        if rc:
            raise RuntimeError(f"hipModuleGetFunction failed: {rc}")
        return fn

    def launch(self, name, n, pointers, stream=0):
        """pointers: buffer name -> device address (int)."""
        k = self.kernels[name]
        items = evaluate_grid(k["grid"][0], n)
        block = k["block"][0]
        assert items % block == 0 and k["block"][1:] == [1, 1]
        # the manifest's grid is 1-D, and a dispatch holds at most 2^32 - 1
        # work-items per dimension (a larger one would be cut short)
        if items > 0xFFFFFFFF:
            raise ValueError(f"{name}: {items} work-items for n = {n} pass "
                             "the 2^32 - 1 one grid dimension holds")
        args = bytearray(k["kernarg_size"])
        for a in k["args"]:
            assert a["type"] == "ptr" and a["size"] == 8
            struct.pack_into("<Q", args, a["offset"], pointers[a["name"]])
        buf = (ctypes.c_char * len(args)).from_buffer(args)
        size = ctypes.c_size_t(len(args))
        extra = (ctypes.c_void_p * 5)(1, ctypes.addressof(buf), 2,
                                      ctypes.addressof(size), 3)
        rc = hip().hipModuleLaunchKernel(self._function(k), items // block, 1,
                                         1, block, 1, 1, 0, stream, None,
                                         extra)
        if rc:
            raise RuntimeError(f"hipModuleLaunchKernel failed: {rc}")

    def close(self):
        for mod in self._modules.values():
            hip().hipModuleUnload(mod)
        self._modules.clear()
