#pragma once

// Persistent cache of compiled code objects across processes.
//
// The reference keeps compiled PTX in memory only, keyed by the full source
// and options (reference src/cuda_jit.cpp:358-378), so every new process pays
// the compile again.  Here a code object can also be written to a directory
// ($PORCH_CACHE_DIR, or one set through the C ABI; off otherwise) as one
// file per key, and later processes read it back.  The key is
// the in-memory cache key (source + options) extended with the hiprtc
// version; each file stores the full key and a checksum of the code, both
// verified on read, and is written to a temporary name and renamed into
// place, so concurrent processes never see a partial file.

#include <optional>
#include <string>

namespace porch::rt::disk {

    // Code bytes stored for `key`, if a valid entry exists.
    std::optional<std::string> load(const std::string& key);
    // Stores `code` for `key` (best effort: failures leave the cache as is).
    void store(const std::string& key, const std::string& code);

    // The directory in use ("" when the cache is off).
    std::string directory();
    // Sets the directory; "" turns the cache off.  Overrides the
    // environment for the rest of the process.
    void set_directory(const std::string& dir);

} // namespace porch::rt::disk
