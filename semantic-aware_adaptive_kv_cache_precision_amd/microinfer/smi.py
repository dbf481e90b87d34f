"""The device's own account of its memory and its users, through amdsmi.

Drop-in for the reference's NVML reader (src/microinfer/nvml.py): the same
functions, read from AMD's System Management Interface instead of NVML, for
the pressure monitor's two readings (monitor.py:147-163: the device's free
memory, and the split of its used memory between this process and the rest)
and the records that name the device. A caller that imported `nvml` imports
this module in its place (`from microinfer import smi as nvml`).

The GPU read is the one HIP runs on, found by its PCI bus id, not by index:
amdsmi lists every GPU of the host, and a process may see only some of them.
amdsmi needs no HIP context; finding the bus id does make one (the first
call of the library does that anyway).
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from functools import cache
from typing import Literal


class SmiUnavailable(RuntimeError):
    """No amdsmi to read from, or it does not know the device."""


#: The reference's name for the same failure, for callers that catch it.
NvmlUnavailable = SmiUnavailable


@dataclass(frozen=True)
class Memory:
    """VRAM in bytes, as the driver accounts for it."""

    total: int
    free: int
    used: int


@dataclass(frozen=True)
class GpuProcess:
    pid: int
    name: str | None        # None where the driver does not name it
    kind: Literal["compute"]
    used_bytes: int | None  # None where the driver does not report it


def _smi():
    try:
        import amdsmi
    except ImportError as exc:  # pragma: no cover - the image ships it
        raise SmiUnavailable("the amdsmi package is not importable") from exc
    return amdsmi


def _bus_id_key(bdf: str) -> str:
    """A PCI address in one spelling: lower case, domain included."""
    bdf = bdf.strip().lower()
    return bdf if bdf.count(":") == 2 else "0000:" + bdf


@cache
def _device():
    """amdsmi's handle for the GPU HIP computes on."""
    smi = _smi()
    try:
        smi.amdsmi_init(smi.AmdSmiInitFlags.INIT_AMD_GPUS)
    except Exception as exc:  # noqa: BLE001 - any init failure means no reader
        raise SmiUnavailable(f"amdsmi_init failed: {exc}") from exc
    from . import _microinfer
    want = _bus_id_key(_microinfer.device_pci_bus_id())
    for handle in smi.amdsmi_get_processor_handles():
        try:
            if _bus_id_key(smi.amdsmi_get_gpu_device_bdf(handle)) == want:
                return smi, handle
        except Exception:  # noqa: BLE001 - a GPU we cannot ask is not ours
            continue
    raise SmiUnavailable(f"amdsmi lists no GPU at {want}, the device HIP runs on")


#: Where memory() read: "amdsmi", or "hip" where amdsmi gives no VRAM
#: account (see memory()).
_source = {"memory": None}


def _hip_memory() -> Memory:
    from . import _microinfer
    info = _microinfer.device_memory_info()
    return Memory(total=int(info["total"]), free=int(info["free"]),
                  used=int(info["total"]) - int(info["free"]))


def memory() -> Memory:
    """Total, free and used VRAM of the device, by amdsmi's account.

    Where amdsmi cannot see the device's VRAM use (inside some containers it
    reports none used while this very process holds device memory), the
    driver's account through HIP (hipMemGetInfo, the KFD's free memory,
    device-wide like amdsmi's) is read instead; memory_source() says which."""
    smi, handle = _device()
    try:
        total = int(smi.amdsmi_get_gpu_memory_total(handle, smi.AmdSmiMemoryType.VRAM))
        used = int(smi.amdsmi_get_gpu_memory_usage(handle, smi.AmdSmiMemoryType.VRAM))
    except Exception:  # noqa: BLE001 - no account from amdsmi: the driver's
        total, used = 0, 0
    hip = _hip_memory()
    # This process holds device memory (its context at least): a reading of
    # none used is amdsmi not seeing the VRAM, not an idle device.
    if total <= 0 or (used == 0 and hip.used > (64 << 20)):
        _source["memory"] = "hip"
        return hip
    _source["memory"] = "amdsmi"
    return Memory(total=total, free=total - used, used=used)


def memory_source() -> str | None:
    """Which account the last memory() read: "amdsmi" or "hip"."""
    return _source["memory"]


def device_name() -> str:
    smi, handle = _device()
    info = smi.amdsmi_get_gpu_asic_info(handle)
    return str(info.get("market_name") or info.get("name") or "AMD GPU")


def driver_version() -> str:
    smi, handle = _device()
    return str(smi.amdsmi_get_gpu_driver_info(handle).get("driver_version", ""))


def _field(entry, name):
    """A process entry's field: amdsmi returns dicts or structures by
    version."""
    if isinstance(entry, dict):
        return entry.get(name)
    return getattr(entry, name, None)


def processes() -> list[GpuProcess]:
    """Every process holding the device's memory, this one included."""
    smi, handle = _device()
    found = []
    for entry in smi.amdsmi_get_gpu_process_list(handle):
        pid = _field(entry, "pid")
        if pid is None:
            continue
        usage = _field(entry, "memory_usage") or {}
        vram = usage.get("vram_mem") if isinstance(usage, dict) else _field(usage, "vram_mem")
        name = _field(entry, "name")
        found.append(GpuProcess(int(pid), str(name) if name else None, "compute",
                                None if vram is None else int(vram)))
    return found


def other_processes() -> list[GpuProcess]:
    """processes(), without this one."""
    own = os.getpid()
    return [p for p in processes() if p.pid != own]


def own_used_bytes() -> int:
    """VRAM this process holds, by the driver's per-process account: no other
    process moves it, so a change in it is this process's own."""
    own = os.getpid()
    for p in processes():
        if p.pid == own:
            if p.used_bytes is None:
                raise SmiUnavailable("the driver does not report this process's memory")
            return p.used_bytes
    return 0


def settled_own_used_bytes() -> int:
    """own_used_bytes() once this process's device context exists and its
    dropped buffers are collected, so that a difference of two readings is
    what happened between them."""
    import gc

    from . import _microinfer
    _microinfer.device_memory_info()
    gc.collect()
    return own_used_bytes()


def others_used_bytes() -> int:
    """What every other process holds, where the driver reports it."""
    return sum(p.used_bytes or 0 for p in other_processes())


def performance_state() -> int | None:
    """Not reported by amdsmi in the reference's P-state terms: None, as the
    reference gives for a GPU that does not report it."""
    return None


def clocks() -> dict[str, int | None]:
    """The current graphics (GFX) and memory (MEM) clocks in MHz; None for a
    clock amdsmi does not give. The reference's "sm" clock is the GFX one on
    AMD GPUs."""
    smi, handle = _device()
    found: dict[str, int | None] = {}
    for domain, kind in (("graphics", "GFX"), ("sm", "GFX"), ("memory", "MEM")):
        try:
            info = smi.amdsmi_get_clk_freq(handle, getattr(smi.AmdSmiClkType, kind))
            current = info["frequency"][info["current"]]
            found[domain] = int(current) // 1_000_000 if current > 100_000 else int(current)
        except Exception:  # noqa: BLE001 - a clock not reported is None
            found[domain] = None
    return found


@dataclass(frozen=True)
class MemorySplit:
    """This process's device memory and every other process's (monitor.py's
    split); None where the driver cannot give one."""

    own_bytes: int | None
    others_bytes: int | None


def headroom() -> int:
    """The device's free memory, the pressure monitor's reading
    (monitor.py:147-149)."""
    return memory().free


def split() -> MemorySplit:
    """monitor.py:152-163's split: own 0 if the driver does not list this
    process, None if a query fails."""
    def read(query):
        try:
            return query()
        except Exception:  # noqa: BLE001 - a split the driver cannot give is None
            return None

    return MemorySplit(read(own_used_bytes), read(others_used_bytes))
