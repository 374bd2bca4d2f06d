# Builds build/libsardyne.so (gfx950 kernels + C host) and the test oracle.
all:
	python -m sardyne_amd.build
	$(MAKE) -C oracle
	@if [ -d /root/reference/csrc ]; then $(MAKE) -C oracle ref; fi
.PHONY: all
