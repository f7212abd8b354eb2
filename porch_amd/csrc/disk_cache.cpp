#include "disk_cache.hpp"

#include <sys/stat.h>
#include <unistd.h>

#include <atomic>
#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>

namespace porch::rt::disk {

    namespace {
        constexpr char magic[8] = {'P', 'O', 'R', 'C', 'H', 'C', 'O', '1'};

        uint64_t fnv1a(const std::string& bytes, uint64_t h = 1469598103934665603ULL) {
            for (const unsigned char c : bytes) {
                h ^= c;
                h *= 1099511628211ULL;
            }
            return h;
        }

        std::string hex(uint64_t v) {
            char text[17];
            std::snprintf(text, sizeof text, "%016llx", static_cast<unsigned long long>(v));
            return text;
        }

        // mkdir -p; true when the directory exists afterwards.
        bool make_directories(const std::string& path) {
            if (path.empty()) return false;
            std::string partial;
            for (size_t i = 0; i < path.size(); ++i) {
                partial += path[i];
                if ((path[i] == '/' && i > 0) || i + 1 == path.size()) {
                    if (::mkdir(partial.c_str(), 0755) != 0 && errno != EEXIST) return false;
                }
            }
            struct stat info {};
            return ::stat(path.c_str(), &info) == 0 && S_ISDIR(info.st_mode);
        }

        // Opt-in: the cache is on when PORCH_CACHE_DIR names a directory.
        std::string default_directory() {
            if (const char* dir = std::getenv("PORCH_CACHE_DIR"); dir != nullptr && *dir != '\0')
                return dir;
            return "";
        }

        struct state {
            std::mutex mutex;
            bool chosen = false;
            std::string dir; // "" = off
        };
        state& current() {
            static state* instance = new state();
            return *instance;
        }

        std::string path_for(const std::string& dir, const std::string& key) {
            return dir + "/" + hex(fnv1a(key)) + hex(fnv1a(key, 0x9E3779B97F4A7C15ULL)) + ".co";
        }

        bool write_all(std::FILE* f, const void* data, size_t size) {
            return size == 0 || std::fwrite(data, 1, size, f) == size;
        }
    } // namespace

    std::string directory() {
        state& s = current();
        std::scoped_lock lock{s.mutex};
        if (!s.chosen) {
            s.dir = default_directory();
            if (!s.dir.empty() && !make_directories(s.dir)) s.dir.clear();
            s.chosen = true;
        }
        return s.dir;
    }

    void set_directory(const std::string& dir) {
        state& s = current();
        std::scoped_lock lock{s.mutex};
        s.dir = dir;
        if (!s.dir.empty() && !make_directories(s.dir)) s.dir.clear();
        s.chosen = true;
    }

    std::optional<std::string> load(const std::string& key) {
        const std::string dir = directory();
        if (dir.empty()) return std::nullopt;
        std::FILE* f = std::fopen(path_for(dir, key).c_str(), "rb");
        if (f == nullptr) return std::nullopt;
        std::optional<std::string> result;
        char head[8];
        uint64_t sizes[3] = {0, 0, 0}; // key size, code size, code checksum
        if (std::fread(head, 1, 8, f) == 8 && std::memcmp(head, magic, 8) == 0 &&
            std::fread(sizes, sizeof(uint64_t), 3, f) == 3 && sizes[0] == key.size() &&
            sizes[1] > 0 && sizes[1] < (uint64_t{1} << 30)) {
            std::string stored_key(sizes[0], '\0');
            std::string code(sizes[1], '\0');
            if (std::fread(stored_key.data(), 1, stored_key.size(), f) == stored_key.size() &&
                stored_key == key && std::fread(code.data(), 1, code.size(), f) == code.size() &&
                fnv1a(code) == sizes[2])
                result = std::move(code);
        }
        std::fclose(f);
        return result;
    }

    void store(const std::string& key, const std::string& code) {
        const std::string dir = directory();
        if (dir.empty() || code.empty()) return;
        static std::atomic<uint64_t> serial{0};
        const std::string final_path = path_for(dir, key);
        const std::string temp = final_path + ".tmp." + std::to_string(::getpid()) + "." +
                                 std::to_string(serial.fetch_add(1));
        std::FILE* f = std::fopen(temp.c_str(), "wb");
        if (f == nullptr) return;
        const uint64_t sizes[3] = {key.size(), code.size(), fnv1a(code)};
        bool ok = write_all(f, magic, 8) && write_all(f, sizes, sizeof sizes) &&
                  write_all(f, key.data(), key.size()) && write_all(f, code.data(), code.size());
        ok = (std::fclose(f) == 0) && ok;
        if (!ok || std::rename(temp.c_str(), final_path.c_str()) != 0) std::remove(temp.c_str());
    }

} // namespace porch::rt::disk
