"""Paged attention kernels (HIP, gfx950) behind the reference's function API."""
