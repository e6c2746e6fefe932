function burgers1d_d(loss, lossd, u, ud, un, und, nu, nud, dt, dtd, dx, dxd, tend, tendd, n, nsteps)
    cadvd = (0.5 * dtd) / dx + -((0.5 * dt) / dx ^ 2) * dxd
    cadv = 0.5 * dt / dx
    __cse_0 = dx * dx
    cdifd = (dt * nud + nu * dtd) / __cse_0 + -((nu * dt) / __cse_0 ^ 2) * (dx * dxd + dx * dxd)
    cdif = nu * dt / __cse_0
    tcd = 0.0
    tc = 0.0
    for i_t = 1:nsteps
        if tc < tend
            for i_x = 1:n
                im = mod(i_x - 2, n) + 1
                ip = mod(i_x, n) + 1
                ucd = ud[i_x]
                uc = u[i_x]
                __cse_1 = u[ip] - u[im]
                __cse_2 = u[ip] - 2.0 * uc + u[im]
                und[i_x] = (ucd + -((uc * __cse_1) * cadvd + (cadv * __cse_1) * ucd + (cadv * uc) * (ud[ip] + -(ud[im])))) + (__cse_2 * cdifd + cdif * ((ud[ip] + -(2.0 * ucd)) + ud[im]))
                un[i_x] = uc - cadv * uc * __cse_1 + cdif * __cse_2
            end
            for i_x2 = 1:n
                ud[i_x2] = und[i_x2]
                u[i_x2] = un[i_x2]
            end
            tcd = tcd + dtd
            tc = tc + dt
        end
    end
    for i_k = 1:n
        __cse_3 = u[i_k]
        lossd[1] = lossd[1] + (2__cse_3) * ud[i_k]
        loss[1] = loss[1] + __cse_3 ^ 2
    end
    return nothing
end

function burgers1d(loss, u, un, nu, dt, dx, tend, n, nsteps)
    cadv = 0.5 * dt / dx
    cdif = nu * dt / (dx * dx)
    tc = 0.0
    for i_t = 1:nsteps
        if tc < tend
            for i_x = 1:n
                im = mod(i_x - 2, n) + 1
                ip = mod(i_x, n) + 1
                uc = u[i_x]
                un[i_x] = uc - cadv * uc * (u[ip] - u[im]) + cdif * (u[ip] - 2.0 * uc + u[im])
            end
            for i_x2 = 1:n
                u[i_x2] = un[i_x2]
            end
            tc = tc + dt
        end
    end
    for i_k = 1:n
        loss[1] = loss[1] + u[i_k] ^ 2
    end
    return nothing
end
