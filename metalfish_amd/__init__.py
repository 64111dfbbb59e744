"""metalfish_amd -- MI355X (gfx950) transformer evaluation backend for MetalFish.

Native pieces (built in-tree by ``__graft_entry__.build()``):

* ``libmfhip.so``   gfx950 kernels + the C ABI of ``include/mfhip.h``;
* ``libmfadapter.so`` the C++ ``HipNetwork`` implementing MetalFish's
  ``NN::Network`` on top of that ABI;
* ``libmfhost.so``  seeded nets and chess positions (``include/mfh_synth.h``).

Python modules: ``backend`` (ctypes binding of the C ABI), ``synth``
(benchmark nets and positions).
"""

__all__ = ["backend", "synth"]
