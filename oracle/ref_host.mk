# Builds oracle/_ref/libref_host.so from the reference's host-only headers in
# place (test infrastructure; skipped by the build when /root/reference is absent).
REF ?= /root/reference
CXX ?= g++

_ref/libref_host.so: ref_host.cpp
	mkdir -p _ref
	$(CXX) -O2 -std=c++17 -fPIC -shared -x c++ -I$(REF)/include -o $@ ref_host.cpp

.PHONY: all
all: _ref/libref_host.so
