! fortai_hip_pack_cache.f90 -- repacked-weight cache files for Fortran hosts.
!
! The reference names a pack file by model / backend / variant / ABI version
! (src/fortai_cache.f90:6-31: pack_key_t, cache_path).  This module builds
! this backend's key and path with those two (it uses the reference's
! fortai_cache module, so the path rule is the reference's own) and reads and
! writes the file this backend stores there: per Q8_0 matrix, the resident
! planes that fortai_hip_q8_weights_pack copies out, so that a later load
! uploads them with fortai_hip_q8_weights_upload_packed instead of repacking.
!
! File layout (little-endian; the same file fortai_amd/pack_cache.py reads
! and writes): "FHIPPACK", u32 format 1, the 32-byte SHA-256 of the first MiB
! of the GGUF the planes came from, u32 record count; per record: u32 name
! length, the name, u32 rows, u32 width, u64 plane bytes, the planes.  A file
! whose digest differs from the GGUF being loaded is stale and is not used.
!
! Errors: FORTAI_INVALID for bad arguments (empty names, unopened files,
! invalid weights), FORTAI_UNSUPPORTED for I/O failures and, on open for
! reading, a missing, foreign or stale file (the caller then repacks and
! writes a new one).
module fortai_hip_pack_cache
    use, intrinsic :: iso_c_binding, only: c_char, c_int, c_int8_t, c_loc, c_null_char, c_ptr, c_size_t
    use, intrinsic :: iso_fortran_env, only: int32, int64
    use fortai_status, only: FORTAI_INVALID, FORTAI_UNSUPPORTED, status_t
    use fortai_cache, only: pack_key_t, cache_path
    use fortai_backend_hip, only: hip_q8_context_t, hip_q8_weights_t, hip_q8_pack_bytes
    implicit none
    private

    character(len=*), parameter, public :: HIP_PACK_BACKEND = 'hip-gfx950'
    character(len=*), parameter, public :: HIP_PACK_VARIANT = 'q8-lanes'
    integer(int32), parameter, public :: HIP_PACK_ABI = 1_int32
    character(len=8), parameter :: MAGIC = 'FHIPPACK'
    integer(int32), parameter :: FORMAT_VERSION = 1_int32
    integer(int64), parameter :: DIGEST_SPAN = 1048576_int64
    ! 1-based stream position of the record count
    integer(int64), parameter :: COUNT_POS = 8_int64 + 4_int64 + 32_int64 + 1_int64

    type, public :: hip_pack_writer_t
        integer :: unit = -1
        integer(int32) :: count = 0_int32
        character(len=:), allocatable :: path
    contains
        procedure :: open => writer_open
        procedure :: add => writer_add
        procedure :: close => writer_close
    end type hip_pack_writer_t

    type, public :: hip_pack_reader_t
        integer :: unit = -1
        character(len=:), allocatable :: names(:)
        integer(int32), allocatable :: rows(:), widths(:)
        integer(int64), allocatable :: offsets(:), sizes(:)
    contains
        procedure :: open => reader_open
        procedure :: has => reader_has
        procedure :: upload => reader_upload
        procedure :: close => reader_close
    end type hip_pack_reader_t

    public :: hip_pack_key, hip_pack_path, hip_gguf_digest

    interface
        ! OpenSSL libcrypto: one-shot SHA-256
        type(c_ptr) function c_sha256(data, n, md) bind(C, name='SHA256')
            import :: c_ptr, c_size_t
            type(c_ptr), value :: data, md
            integer(c_size_t), value :: n
        end function
        integer(c_int) function c_mkdir(path, mode) bind(C, name='mkdir')
            import :: c_char, c_int
            character(kind=c_char), intent(in) :: path(*)
            integer(c_int), value :: mode
        end function
        integer(c_int) function c_rename(old, new) bind(C, name='rename')
            import :: c_char, c_int
            character(kind=c_char), intent(in) :: old(*), new(*)
        end function
    end interface

contains

    ! This backend's pack key for a model name (any non-empty text, e.g. the
    ! GGUF's stem).
    function hip_pack_key(model) result(key)
        character(len=*), intent(in) :: model
        type(pack_key_t) :: key

        key%model = trim(model)
        key%backend = HIP_PACK_BACKEND
        key%variant = HIP_PACK_VARIANT
        key%abi_version = HIP_PACK_ABI
    end function hip_pack_key

    ! root/model/hip-gfx950-q8-lanes-abi1.pack, by the reference's cache_path
    ! (root/invalid.pack for an empty model name).
    function hip_pack_path(root, model) result(path)
        character(len=*), intent(in) :: root, model
        character(len=:), allocatable :: path

        path = cache_path(root, hip_pack_key(model))
    end function hip_pack_path

    ! SHA-256 of the first MiB (or the whole file, if shorter) of a GGUF.
    subroutine hip_gguf_digest(gguf_path, digest, stat)
        character(len=*), intent(in) :: gguf_path
        integer(c_int8_t), target, intent(out) :: digest(32)
        type(status_t), intent(out) :: stat
        integer(c_int8_t), allocatable, target :: head(:)
        integer(int64) :: file_size
        integer :: u, ios
        type(c_ptr) :: ignored

        call stat%clear()
        digest = 0_c_int8_t
        inquire (file=gguf_path, size=file_size)
        if (file_size < 0_int64) then
            call stat%set(FORTAI_UNSUPPORTED, 'pack digest: cannot read ' // gguf_path)
            return
        end if
        allocate (head(max(1_int64, min(file_size, DIGEST_SPAN))))
        open (newunit=u, file=gguf_path, access='stream', form='unformatted', status='old', action='read', &
            iostat=ios)
        if (ios == 0) read (u, iostat=ios) head(1:min(file_size, DIGEST_SPAN))
        if (ios == 0) close (u)
        if (ios /= 0) then
            call stat%set(FORTAI_UNSUPPORTED, 'pack digest: cannot read ' // gguf_path)
            return
        end if
        ignored = c_sha256(c_loc(head), int(min(file_size, DIGEST_SPAN), c_size_t), c_loc(digest))
    end subroutine hip_gguf_digest

    ! ---- writer ------------------------------------------------------------------

    ! Start a pack at path (written to path.part, renamed over path on close),
    ! creating the directories on the way.
    subroutine writer_open(self, path, digest, stat)
        class(hip_pack_writer_t), intent(inout) :: self
        character(len=*), intent(in) :: path
        integer(c_int8_t), intent(in) :: digest(32)
        type(status_t), intent(out) :: stat
        integer :: ios

        call stat%clear()
        if (self%unit /= -1 .or. len_trim(path) == 0) then
            call stat%set(FORTAI_INVALID, 'pack writer: already open, or empty path')
            return
        end if
        call make_parents(trim(path))
        self%path = trim(path)
        self%count = 0_int32
        open (newunit=self%unit, file=self%path // '.part', access='stream', form='unformatted', &
            status='replace', action='write', iostat=ios)
        if (ios == 0) write (self%unit, iostat=ios) MAGIC, FORMAT_VERSION, digest, 0_int32
        if (ios /= 0) then
            call abandon(self)
            call stat%set(FORTAI_UNSUPPORTED, 'pack writer: cannot write ' // trim(path) // '.part')
        end if
    end subroutine writer_open

    ! Append one matrix's resident planes under a name.
    subroutine writer_add(self, name, weights, rows, width, stat)
        class(hip_pack_writer_t), intent(inout) :: self
        character(len=*), intent(in) :: name
        type(hip_q8_weights_t), intent(in) :: weights
        integer, intent(in) :: rows, width
        type(status_t), intent(out) :: stat
        integer(c_int8_t), allocatable, target :: planes(:)
        integer(c_size_t) :: bytes
        integer :: ios

        call stat%clear()
        bytes = hip_q8_pack_bytes(rows, width)
        if (self%unit == -1 .or. len_trim(name) == 0 .or. bytes == 0_c_size_t) then
            call stat%set(FORTAI_INVALID, 'pack writer: not open, empty name or invalid shape')
            return
        end if
        allocate (planes(bytes))
        call weights%pack(planes, stat)
        if (.not. stat%is_ok()) return
        write (self%unit, iostat=ios) int(len_trim(name), int32), trim(name), int(rows, int32), &
            int(width, int32), int(bytes, int64), planes
        if (ios /= 0) then
            call stat%set(FORTAI_UNSUPPORTED, 'pack writer: write failed for ' // trim(name))
            return
        end if
        self%count = self%count + 1_int32
    end subroutine writer_add

    ! Write the record count and move the finished file into place.
    subroutine writer_close(self, stat)
        class(hip_pack_writer_t), intent(inout) :: self
        type(status_t), intent(out) :: stat
        integer :: ios

        call stat%clear()
        if (self%unit == -1) return
        write (self%unit, pos=COUNT_POS, iostat=ios) self%count
        if (ios == 0) close (self%unit, iostat=ios)
        self%unit = -1
        if (ios == 0) then
            if (c_rename(self%path // '.part' // c_null_char, self%path // c_null_char) /= 0_c_int) ios = 1
        end if
        if (ios /= 0) call stat%set(FORTAI_UNSUPPORTED, 'pack writer: cannot finish ' // self%path)
    end subroutine writer_close

    subroutine abandon(self)
        type(hip_pack_writer_t), intent(inout) :: self
        integer :: ios
        if (self%unit /= -1) close (self%unit, status='delete', iostat=ios)
        self%unit = -1
    end subroutine abandon

    ! mkdir of every directory on the way to path's last component (existing
    ! ones are left as they are).
    subroutine make_parents(path)
        character(len=*), intent(in) :: path
        integer :: i
        integer(c_int) :: ignored

        do i = 2, len(path)
            if (path(i:i) == '/') ignored = c_mkdir(path(1:i - 1) // c_null_char, int(o'755', c_int))
        end do
    end subroutine make_parents

    ! ---- reader ------------------------------------------------------------------

    ! Open a pack and read its index.  FORTAI_UNSUPPORTED if the file is
    ! missing, is not a pack of this format, or was made from another GGUF.
    subroutine reader_open(self, path, digest, stat)
        class(hip_pack_reader_t), intent(inout) :: self
        character(len=*), intent(in) :: path
        integer(c_int8_t), intent(in) :: digest(32)
        type(status_t), intent(out) :: stat
        character(len=8) :: magic_in
        character(len=:), allocatable :: name
        integer(c_int8_t) :: digest_in(32)
        integer(int32) :: version, count, name_len, r, w
        integer(int64) :: bytes, here, file_size
        integer :: ios, i, longest
        logical :: exists, intact

        call stat%clear()
        call self%close()
        inquire (file=path, exist=exists)
        if (.not. exists) then
            call stat%set(FORTAI_UNSUPPORTED, 'pack reader: no pack at ' // trim(path))
            return
        end if
        open (newunit=self%unit, file=path, access='stream', form='unformatted', status='old', action='read', &
            iostat=ios)
        if (ios == 0) read (self%unit, iostat=ios) magic_in, version, digest_in, count
        if (ios /= 0 .or. magic_in /= MAGIC .or. version /= FORMAT_VERSION .or. count < 0_int32) then
            call self%close()
            call stat%set(FORTAI_UNSUPPORTED, 'pack reader: not a pack of this format: ' // trim(path))
            return
        end if
        if (any(digest_in /= digest)) then
            call self%close()
            call stat%set(FORTAI_UNSUPPORTED, 'pack reader: stale pack (made from another GGUF): ' // trim(path))
            return
        end if
        ! first pass: check the record sizes against the file, find the longest
        ! name; second pass: the index
        inquire (unit=self%unit, size=file_size)
        longest = 1
        here = COUNT_POS + 4_int64
        intact = .true.
        do i = 1, count
            if (here + 20_int64 > file_size + 1_int64) then
                intact = .false.
                exit
            end if
            read (self%unit, pos=here, iostat=ios) name_len
            if (ios == 0 .and. name_len > 0_int32) &
                read (self%unit, pos=here + 4_int64 + name_len + 8_int64, iostat=ios) bytes
            if (ios /= 0 .or. name_len <= 0_int32 .or. bytes < 0_int64) then
                intact = .false.
                exit
            end if
            longest = max(longest, int(name_len))
            here = here + 4_int64 + name_len + 16_int64 + bytes
        end do
        if (.not. intact .or. here /= file_size + 1_int64) then
            call self%close()
            call stat%set(FORTAI_UNSUPPORTED, 'pack reader: truncated pack: ' // trim(path))
            return
        end if
        allocate (character(len=longest) :: self%names(count))
        allocate (self%rows(count), self%widths(count), self%offsets(count), self%sizes(count))
        here = COUNT_POS + 4_int64
        do i = 1, count
            read (self%unit, pos=here) name_len
            allocate (character(len=name_len) :: name)
            read (self%unit) name, r, w, bytes
            self%names(i) = name
            deallocate (name)
            self%rows(i) = r
            self%widths(i) = w
            self%sizes(i) = bytes
            self%offsets(i) = here + 4_int64 + name_len + 16_int64
            here = self%offsets(i) + bytes
        end do
    end subroutine reader_open

    ! Index of a record by name (0 if absent).
    integer function reader_has(self, name) result(index)
        class(hip_pack_reader_t), intent(in) :: self
        character(len=*), intent(in) :: name
        integer :: i

        index = 0
        if (.not. allocated(self%names)) return
        do i = 1, size(self%names)
            if (self%names(i) == name) then
                index = i
                return
            end if
        end do
    end function reader_has

    ! Create a resident matrix from the named record.  FORTAI_INVALID if the
    ! record is absent or its shape differs from the one asked for.
    subroutine reader_upload(self, name, context, weights, rows, width, stat)
        class(hip_pack_reader_t), intent(inout) :: self
        character(len=*), intent(in) :: name
        type(hip_q8_context_t), intent(in) :: context
        type(hip_q8_weights_t), intent(inout) :: weights
        integer, intent(in) :: rows, width
        type(status_t), intent(out) :: stat
        integer(c_int8_t), allocatable :: planes(:)
        integer :: i, ios

        call stat%clear()
        i = self%has(name)
        if (self%unit == -1 .or. i == 0) then
            call stat%set(FORTAI_INVALID, 'pack reader: no record ' // trim(name))
            return
        end if
        if (self%rows(i) /= rows .or. self%widths(i) /= width .or. &
                self%sizes(i) /= int(hip_q8_pack_bytes(rows, width), int64)) then
            call stat%set(FORTAI_INVALID, 'pack reader: record ' // trim(name) // ' has another shape')
            return
        end if
        allocate (planes(self%sizes(i)))
        read (self%unit, pos=self%offsets(i), iostat=ios) planes
        if (ios /= 0) then
            call stat%set(FORTAI_UNSUPPORTED, 'pack reader: read failed for ' // trim(name))
            return
        end if
        call weights%upload_packed(context, planes, rows, width, stat)
    end subroutine reader_upload

    subroutine reader_close(self)
        class(hip_pack_reader_t), intent(inout) :: self
        integer :: ios

        if (self%unit /= -1) close (self%unit, iostat=ios)
        self%unit = -1
        if (allocated(self%names)) deallocate (self%names)
        if (allocated(self%rows)) deallocate (self%rows, self%widths, self%offsets, self%sizes)
    end subroutine reader_close

end module fortai_hip_pack_cache
