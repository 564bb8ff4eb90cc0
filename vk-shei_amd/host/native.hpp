// C++ ownership of a libmslim_attn context, the way native_hip.rs wraps the
// reference bridge: one handle, serialised use, and every nonzero return
// turned into an error "{stage} failed: code={code}: {details}"
// (native_hip.rs:38-49).
#pragma once

#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>

#include "../../include/mslim_attn.h"

namespace mslim {

// anyhow-style error carrying the reference's message text.
class Error : public std::runtime_error {
public:
    explicit Error(const std::string &message) : std::runtime_error(message) {}
};

// Throws Error(message) unless `condition` holds (anyhow::ensure!).
inline void ensure(bool condition, const std::string &message) {
    if (!condition) throw Error(message);
}

class NativeError : public Error {
public:
    NativeError(const std::string &stage, int code, const std::string &details)
        : Error(stage + " failed: code=" + std::to_string(code) + ": " + details),
          stage_(stage), code_(code), details_(details) {}
    const std::string &stage() const { return stage_; }
    int code() const { return code_; }
    const std::string &details() const { return details_; }

private:
    std::string stage_;
    int code_;
    std::string details_;
};

// Shared handle: HipRuntime's Arc<Mutex<Inner>> (native_hip.rs:58-61).
class NativeContext {
public:
    static std::shared_ptr<NativeContext> create() {
        void *h = mslim_attn_ctx_new();
        if (!h) throw NativeError("mslim_attn_ctx_new", 0, mslim_attn_last_error());
        return std::shared_ptr<NativeContext>(new NativeContext(h));
    }
    // A context owned elsewhere (for example by a Python caller); it is not
    // destroyed with this object.
    static std::shared_ptr<NativeContext> borrow(void *handle) {
        auto c = std::shared_ptr<NativeContext>(new NativeContext(handle));
        c->owned_ = false;
        return c;
    }
    ~NativeContext() {
        if (owned_) mslim_attn_ctx_destroy(handle_);
    }
    NativeContext(const NativeContext &) = delete;
    NativeContext &operator=(const NativeContext &) = delete;

    void *handle() const { return handle_; }
    std::mutex &mutex() { return mutex_; }

    void check(const std::string &stage, int code) const {
        if (code != 0) throw NativeError(stage, code, mslim_attn_last_error());
    }

private:
    explicit NativeContext(void *h) : handle_(h) {}
    void *handle_;
    bool owned_ = true;
    std::mutex mutex_;
};

}  // namespace mslim
